/*
 * hx_host.h — host-side internals of libhearth.so (MI355X verify engine).
 *
 * Container format: docs/FORMAT.md of the reference (engine/src/modelfile.c is its
 * reader there); the weight encodings and the block structs are fixed by FORMAT.md §6.
 */
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "hearth.h"
#include "hearth_gpu.h"

namespace hx {

constexpr int QK = 64;                      /* elements per Q8/Q4 block and activation block */
constexpr uint32_t CANON_NAN = 0x7fc00000u; /* the one NaN bit pattern outputs carry */

/* Error codes (reference engine/src/hx_model.h:60-68). */
enum { OK = 0, E_ARG = -1, E_TOKEN = -2, E_CAPACITY = -3, E_IO = -4, E_NOMEM = -5, E_FORMAT = -6 };

/* Sampler settings check, as Sampler.__post_init__ (python/hearth/generate.py:45-56):
 * OK or E_ARG. */
int check_sampler(const hearth_sampler *s);

enum { ATTN_GQA = 0, ATTN_MLA = 1 };
enum { QKNORM_NONE = 0, QKNORM_HEAD = 1, QKNORM_FULL = 2 };
enum { ROPE_NEOX = 0, ROPE_GPTJ = 1 };
enum { SCORE_SOFTMAX = 0, SCORE_SIGMOID = 1 };

/* ---- formats (FORMAT.md §6) ---- */
size_t row_bytes(int dtype, int64_t n);
bool dtype_is_quant(int dtype);
const char *dtype_name(int dtype);
float f16_to_f32(uint16_t h);
uint16_t f32_to_f16(float f);
uint16_t f32_to_bf16(float f);
float bf16_to_f32(uint16_t h);
void quantize_row(int dtype, const float *src, uint8_t *dst, int64_t n);
void dequantize_row(int dtype, const uint8_t *src, float *dst, int64_t n);

/* ---- container (FORMAT.md §1-5) ---- */
struct Config {
    std::string arch;
    int n_layers = 0, d_model = 0, vocab = 0, max_seq = 4096;
    float eps = 1e-6f;
    int attn_kind = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, qk_norm = 0, qkv_bias = 0;
    int q_lora = 0, kv_lora = 0, nope = 0, rope_qk = 0, v_head = 0, rope_dim = 0, rope_style = 0;
    float rope_factor = 1.0f, attn_scale = 1.0f;
    int dense_ffn = 0, n_experts = 0, top_k = 0, expert_ffn = 0, shared_ffn = 0, shared_gate = 0;
    int score_fn = 0, score_bias = 0, n_group = 1, topk_group = 1, norm_topk = 0;
    float routed_scale = 1.0f, emb_scale = 1.0f, resid_scale = 1.0f, logit_scale = 1.0f;
    int tie = 0;
    std::vector<uint8_t> layer_kind;
    int n_moe = 0;
    int bos_id = -1;
    std::vector<int> eos_ids;
};

struct Tensor {
    std::string name;
    int dtype = 0, ndim = 0;
    int64_t shape[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
};

struct ExpertEntry {
    uint64_t offset = 0, nbytes = 0;
    uint32_t dtype = 0, flags = 0;
};

class ModelFile {
public:
    ~ModelFile();
    /* Parses and validates (bounds, alignment, overlaps, canonical tensor shapes).
     * The file stays mapped read-only; data() points into the mapping. */
    bool open(const std::string &path, std::string &err);
    const Tensor *tensor(const std::string &name) const;
    const Tensor *layer_tensor(int layer, const char *suffix) const;
    const ExpertEntry *expert(int layer, int e) const;
    const uint8_t *data(uint64_t off) const { return map_ + off; }
    uint64_t size() const { return size_; }

    Config cfg;
    std::vector<Tensor> tensors;
    std::vector<ExpertEntry> experts;
    uint64_t dense_bytes = 0, expert_region_bytes = 0, slab_bytes_max = 0;
    double params_total = 0.0, params_active = 0.0;
    std::string path;

private:
    uint8_t *map_ = nullptr;
    uint64_t size_ = 0;
};

/* Slab layout (FORMAT.md §5): returns the padded slab size and the three offsets. */
uint64_t slab_layout(int dtype, int64_t D, int64_t F, uint64_t *og, uint64_t *ou, uint64_t *od);

/* Logging to stderr, level from HEARTH_LOG / verbose. */
void log_msg(int level, const char *fmt, ...);
enum { LOG_ERROR = 0, LOG_WARN = 1, LOG_INFO = 2, LOG_DEBUG = 3 };
void set_log_level(int level);
int get_log_level();

} // namespace hx
