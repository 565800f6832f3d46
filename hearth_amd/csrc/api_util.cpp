/*
 * api_util.cpp — engine-free entry points that run single kernels on the GPU:
 * hearth_matmul (reference engine/src/quant.c:573-600: NUMERICS §3 Y = W X for T
 * rows, the utility the reference's tests use for its pinned kernel hashes) and
 * hearth_gpu_accept_greedy (the acceptance kernel on caller logits).
 */
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <vector>

#include "hearth.h"
#include "hearth_gpu.h"
#include "hx_host.h"
#include "hx_launch.h"

using namespace hx;

namespace {

int device() {
    const char *s = getenv("HEARTH_DEVICE");
    return s && *s ? atoi(s) : 0;
}

/* device buffers freed at scope exit */
struct Scratch {
    std::vector<void *> p;
    hipStream_t st = nullptr;
    bool ok = true;
    void *get(size_t n) {
        void *q = nullptr;
        if (hipMalloc(&q, n ? n : 256) != hipSuccess) { ok = false; return nullptr; }
        p.push_back(q);
        return q;
    }
    ~Scratch() {
        if (st) {
            (void)hipStreamSynchronize(st);
            (void)hipStreamDestroy(st);
        }
        for (void *q : p) (void)hipFree(q);
    }
};

} // namespace

int hx::check_sampler(const hearth_sampler *s) {
    if (!s) return E_ARG;
    if (!std::isfinite(s->temperature) || s->temperature < 0.0) return E_ARG;
    if (s->top_k < 0 || !(s->top_p > 0.0 && s->top_p <= 1.0) || !(s->min_p >= 0.0 && s->min_p <= 1.0)) return E_ARG;
    if (!std::isfinite(s->repetition_penalty) || !(s->repetition_penalty > 0.0)) return E_ARG;
    if (s->n_context < 0 || (s->n_context > 0 && !s->context)) return E_ARG;
    return OK;
}

extern "C" {

/* 0 ok, -1 bad arguments, -2 ISA not available on this CPU, -3 device memory /
 * device error (reference quant.c:573). */
HEARTH_API int hearth_matmul(int dtype, const void *W, int64_t n_rows, int64_t n_cols, const float *X, int T, float *Y,
                             int isa) {
    if (isa < HEARTH_ISA_AUTO || isa > HEARTH_ISA_AVX512) return -1;
    if (dtype < HEARTH_F32 || dtype > HEARTH_U8 || n_rows < 0 || T < 0 || row_bytes(dtype, n_cols) == 0) return -1;
    if (isa != HEARTH_ISA_AUTO && isa > hearth_cpu_isa()) return -2;
    if (dtype > HEARTH_Q4) return -1;   /* no kernel for I32 / U8 */
    if (T == 0 || n_rows == 0) return 0;
    if (!W || !X || !Y) return -1;
    if (n_rows > (1 << 30) || n_cols > (1 << 30)) return -1;
    if (hipSetDevice(device()) != hipSuccess) return -3;
    Scratch s;
    if (hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking) != hipSuccess) return -3;
    const size_t wb = (size_t)n_rows * row_bytes(dtype, n_cols);
    const int rows = (int)n_rows, cols = (int)n_cols;
    uint8_t *dW = (uint8_t *)s.get(wb);
    float *dX = (float *)s.get(sizeof(float) * (size_t)T * cols);
    float *dY = (float *)s.get(sizeof(float) * (size_t)T * rows);
    if (!s.ok) return -3;
    if (hipMemcpyAsync(dW, W, wb, hipMemcpyHostToDevice, s.st) != hipSuccess ||
        hipMemcpyAsync(dX, X, sizeof(float) * (size_t)T * cols, hipMemcpyHostToDevice, s.st) != hipSuccess)
        return -3;
    if (dtype_is_quant(dtype)) {
        hxd::QMat m{};
        m.dtype = dtype;
        m.rows = rows;
        m.rows_pad = (rows + 15) & ~15;
        m.nb = cols / 64;
        m.nbp = (m.nb + 1) & ~1;
        m.w = (const uint8_t *)s.get((size_t)(m.rows_pad / 16) * m.nbp * 1024 / (dtype == HEARTH_Q4 ? 2 : 1));
        m.d = (const uint16_t *)s.get(sizeof(uint16_t) * (size_t)m.nbp * m.rows_pad);
        hxd::Act a{};
        a.nbp = m.nbp;
        a.q = (int8_t *)s.get((size_t)T * a.nbp * 64);
        a.d = (float *)s.get(sizeof(float) * (size_t)T * a.nbp);
        a.s = (int32_t *)s.get(sizeof(int32_t) * (size_t)T * a.nbp);
        if (!s.ok) return -3;
        hxl::repack(dW, 0, m.rows_pad, m, s.st);
        hxl::quant_rows(dX, cols, T, m.nb, a, s.st);
        hxd::GemmArgs g{};
        g.nseg = 1;
        g.seg[0].m = m;
        g.seg[0].Y = dY;
        g.seg[0].ldy = rows;
        g.a = a;
        g.T = T;
        hxl::gemm(g, s.st);
    } else {
        hxl::fgemv(dtype, dW, rows, cols, dX, cols, T, dY, rows, s.st);
    }
    if (hipMemcpyAsync(Y, dY, sizeof(float) * (size_t)T * rows, hipMemcpyDeviceToHost, s.st) != hipSuccess) return -3;
    if (hipStreamSynchronize(s.st) != hipSuccess) return -3;
    return 0;
}

HEARTH_API int hearth_gpu_accept_greedy(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                                        int32_t *path_out, int *n_path, int32_t *final_tok) {
    if (!rows || n < 1 || V < 1 || !tokens || !path_out || !n_path || !final_tok) return E_ARG;
    for (int i = 0; i < n; i++)
        if (parent && ((i == 0 && parent[i] != -1) || (i > 0 && (parent[i] < 0 || parent[i] >= i)))) return E_ARG;
    if (hipSetDevice(device()) != hipSuccess) return E_IO;
    Scratch s;
    if (hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking) != hipSuccess) return E_IO;
    float *dr = (float *)s.get(sizeof(float) * (size_t)n * V);
    int *dt = (int *)s.get(sizeof(int) * (size_t)n * 4 + 16);
    int *dpart = (int *)s.get(sizeof(int) * (size_t)n * hxd::ACCEPT_PARTS * 3);
    if (!s.ok) return E_NOMEM;
    std::vector<int> hp(n);
    for (int i = 0; i < n; i++) hp[i] = parent ? parent[i] : i - 1;
    int *dtok = dt, *dpar = dt + n, *damax = dt + 2 * n, *dpath = dt + 3 * n, *dres = dt + 4 * n;
    if (hipMemcpyAsync(dr, rows, sizeof(float) * (size_t)n * V, hipMemcpyHostToDevice, s.st) != hipSuccess ||
        hipMemcpyAsync(dtok, tokens, sizeof(int) * n, hipMemcpyHostToDevice, s.st) != hipSuccess ||
        hipMemcpyAsync(dpar, hp.data(), sizeof(int) * n, hipMemcpyHostToDevice, s.st) != hipSuccess)
        return E_IO;
    hxd::AcceptArgs a{};
    a.rows = dr; a.n = n; a.V = V; a.tokens = dtok; a.parent = dpar; a.amax = damax; a.path = dpath; a.result = dres;
    a.part_v = (float *)dpart; a.part_i = dpart + (size_t)n * hxd::ACCEPT_PARTS;
    a.part_f = dpart + 2 * (size_t)n * hxd::ACCEPT_PARTS;
    hxl::accept_greedy(a, s.st);
    std::vector<int> res(3), path(n);
    if (hipMemcpyAsync(res.data(), dres, sizeof(int) * 3, hipMemcpyDeviceToHost, s.st) != hipSuccess ||
        hipMemcpyAsync(path.data(), dpath, sizeof(int) * n, hipMemcpyDeviceToHost, s.st) != hipSuccess ||
        hipStreamSynchronize(s.st) != hipSuccess)
        return E_IO;
    if (res[2] != 0) return E_ARG;
    *n_path = res[0];
    for (int j = 0; j < res[0]; j++) path_out[j] = path[j];
    *final_tok = res[1];
    return OK;
}

HEARTH_API int hearth_gpu_accept_sample(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                                        const hearth_sampler *smp, const double *q, const double *u,
                                        int32_t *path_out, int *n_path, int32_t *final_tok) {
    if (!rows || n < 1 || V < 1 || !tokens || !u || !path_out || !n_path || !final_tok) return E_ARG;
    if (check_sampler(smp) != OK || n > hxd::SAMPLE_NMAX || V > hxd::SAMPLE_VMAX) return E_ARG;
    for (int i = 0; i < n; i++) {
        if (tokens[i] < 0 || tokens[i] >= V) return E_TOKEN;
        if (parent && ((i == 0 && parent[i] != -1) || (i > 0 && (parent[i] < 0 || parent[i] >= i)))) return E_ARG;
    }
    if (hipSetDevice(device()) != hipSuccess) return E_IO;
    Scratch s;
    if (hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking) != hipSuccess) return E_IO;
    float *dr = (float *)s.get(sizeof(float) * (size_t)n * V);
    if (!s.ok) return E_NOMEM;
    hxl::SampleScratch m;
    const int n_ctx = smp->repetition_penalty != 1.0 ? smp->n_context : 0;
    if (m.ensure(n, V, q != nullptr, n_ctx) != hipSuccess) return E_NOMEM;
    std::vector<int> hp(n);
    for (int i = 0; i < n; i++) hp[i] = parent ? parent[i] : i - 1;
    if (hipMemcpyAsync(dr, rows, sizeof(float) * (size_t)n * V, hipMemcpyHostToDevice, s.st) != hipSuccess ||
        hipMemcpyAsync(m.tok, tokens, sizeof(int) * n, hipMemcpyHostToDevice, s.st) != hipSuccess ||
        hipMemcpyAsync(m.par, hp.data(), sizeof(int) * n, hipMemcpyHostToDevice, s.st) != hipSuccess)
        return E_IO;
    const hxl::SamplerSpec sp{smp->temperature, smp->top_p, smp->min_p, smp->repetition_penalty, smp->top_k,
                              smp->context, n_ctx};
    if (hxl::accept_sample(m, dr, n, V, m.tok, m.par, sp, q, u, s.st, false, hxl::max_siblings(hp.data(), n)) !=
        hipSuccess)
        return E_IO;
    std::vector<int> res(3), path(n);
    if (hipMemcpyAsync(res.data(), m.result, sizeof(int) * 3, hipMemcpyDeviceToHost, s.st) != hipSuccess ||
        hipMemcpyAsync(path.data(), m.path, sizeof(int) * n, hipMemcpyDeviceToHost, s.st) != hipSuccess ||
        hipStreamSynchronize(s.st) != hipSuccess)
        return E_IO;
    if (res[2] != 0) return E_ARG;
    *n_path = res[0];
    for (int j = 0; j < res[0]; j++) path_out[j] = path[j];
    *final_tok = res[1];
    return OK;
}

HEARTH_API int hearth_gpu_probs(const float *rows, int n, int V, const int32_t *tokens, const int32_t *parent,
                                const hearth_sampler *smp, double *p_out) {
    if (!rows || n < 1 || V < 1 || !tokens || !p_out) return E_ARG;
    if (check_sampler(smp) != OK || n > hxd::SAMPLE_NMAX || V > hxd::SAMPLE_VMAX) return E_ARG;
    for (int i = 0; i < n; i++)
        if (parent && ((i == 0 && parent[i] != -1) || (i > 0 && (parent[i] < 0 || parent[i] >= i)))) return E_ARG;
    if (hipSetDevice(device()) != hipSuccess) return E_IO;
    Scratch s;
    if (hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking) != hipSuccess) return E_IO;
    float *dr = (float *)s.get(sizeof(float) * (size_t)n * V);
    if (!s.ok) return E_NOMEM;
    hxl::SampleScratch m;
    const int n_ctx = smp->repetition_penalty != 1.0 ? smp->n_context : 0;
    if (m.ensure(n, V, false, n_ctx) != hipSuccess) return E_NOMEM;
    std::vector<int> hp(n);
    for (int i = 0; i < n; i++) hp[i] = parent ? parent[i] : i - 1;
    if (hipMemcpyAsync(dr, rows, sizeof(float) * (size_t)n * V, hipMemcpyHostToDevice, s.st) != hipSuccess ||
        hipMemcpyAsync(m.tok, tokens, sizeof(int) * n, hipMemcpyHostToDevice, s.st) != hipSuccess ||
        hipMemcpyAsync(m.par, hp.data(), sizeof(int) * n, hipMemcpyHostToDevice, s.st) != hipSuccess)
        return E_IO;
    const hxl::SamplerSpec sp{smp->temperature, smp->top_p, smp->min_p, smp->repetition_penalty, smp->top_k,
                              smp->context, n_ctx};
    if (hxl::sample_probs(m, dr, n, V, m.tok, m.par, sp, s.st) != hipSuccess) return E_IO;
    std::vector<int> rc(n);
    if (hipMemcpyAsync(rc.data(), m.row_rc, sizeof(int) * n, hipMemcpyDeviceToHost, s.st) != hipSuccess ||
        hipMemcpyAsync(p_out, m.P, sizeof(double) * (size_t)n * V, hipMemcpyDeviceToHost, s.st) != hipSuccess ||
        hipStreamSynchronize(s.st) != hipSuccess)
        return E_IO;
    for (int i = 0; i < n; i++)
        if (rc[i] != 0) return E_ARG;
    return OK;
}

} // extern "C"
