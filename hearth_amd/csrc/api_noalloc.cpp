/*
 * api_noalloc.cpp — hearth_gpu_accept_greedy_noalloc: the greedy acceptance of
 * hearth_gpu_accept_greedy for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops that forbid hipMalloc). Inputs and outputs are the
 * caller's device buffers; the kernels' scratch (per-slice maxima, the row argmaxes and
 * the chain's parent table) lives in `scratch`, a fixed array of this library on every
 * GPU it runs on, held until the process ends.
 *
 * In host code the name `scratch` is a host-side stand-in, not a device address: the
 * device address comes from hipGetSymbolAddress, once per device with that device
 * current, and only that address is handed to kernels. Calls that overlap on one GPU
 * share the array and race; the array keeps the last call's contents, and nothing in it
 * needs to start at zero (every word a kernel reads was written earlier in the call).
 */
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "hearth.h"
#include "hearth_gpu.h"
#include "hx_host.h"
#include "hx_launch.h"

namespace {

constexpr int NOALLOC_ROWS = HEARTH_GPU_NOALLOC_MAX_ROWS;
/* words per row: amax, parent, and ACCEPT_PARTS each of part_v / part_i / part_f */
constexpr size_t WORDS_PER_ROW = 2 + 3 * (size_t)hxd::ACCEPT_PARTS;
constexpr size_t SCRATCH_BYTES = 4 * WORDS_PER_ROW * NOALLOC_ROWS;

__device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

constexpr int MAX_DEV = 64;
std::mutex g_mu;
void *g_ptr[MAX_DEV] = {};

/* device address of `scratch` on device dev (current); nullptr if it cannot be had */
void *scratch_on(int dev) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        g_ptr[dev] = p;
    }
    return g_ptr[dev];
}

/* parent[i] = i - 1: the chain's parent table, written by a kernel (no memset, no copy) */
__global__ void k_chain_parent(int *parent, int n) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) parent[i] = i - 1;
}

} // namespace

extern "C" {

HEARTH_API int hearth_gpu_accept_greedy_noalloc(const float *rows, int n, int V, const int32_t *tokens,
                                                const int32_t *parent, int32_t *path_out, int32_t *result,
                                                void *stream) {
    if (!rows || n < 1 || V < 1 || !tokens || !path_out || !result) return hx::E_ARG;
    if (n > NOALLOC_ROWS) return hx::E_CAPACITY;
    /* a HIP error the calling thread has not read yet is the caller's: it is left in place
     * (not cleared by this call's check below) and nothing is launched */
    if (hipPeekAtLastError() != hipSuccess) return hx::E_IO;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return hx::E_IO;
    unsigned char *base = (unsigned char *)scratch_on(dev);
    if (!base) return hx::E_IO;
    hipStream_t st = (hipStream_t)stream;
    int *w = (int *)base;
    hxd::AcceptArgs a{};
    a.rows = rows;
    a.n = n;
    a.V = V;
    a.tokens = tokens;
    a.amax = w;
    int *par = w + NOALLOC_ROWS;
    a.part_v = (float *)(par + NOALLOC_ROWS);
    a.part_i = (int *)a.part_v + (size_t)NOALLOC_ROWS * hxd::ACCEPT_PARTS;
    a.part_f = a.part_i + (size_t)NOALLOC_ROWS * hxd::ACCEPT_PARTS;
    if (parent) {
        a.parent = parent;
    } else {
        hipLaunchKernelGGL(k_chain_parent, dim3((n + 255) / 256), dim3(256), 0, st, par, n);
        a.parent = par;
    }
    a.path = path_out;
    a.result = result;
    hxl::accept_greedy(a, st);
    return hipGetLastError() == hipSuccess ? hx::OK : hx::E_IO;   /* this call's launches only */
}

} // extern "C"
