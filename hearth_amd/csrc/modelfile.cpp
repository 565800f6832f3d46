/*
 * modelfile.cpp — reader of the .hearth container (the reference's docs/FORMAT.md,
 * version 1; its reader is engine/src/modelfile.c:691-884).
 *
 * The file is mapped read-only and validated before anything uses it: every
 * section, tensor and slab lies inside the file, nothing overlaps (aliased slabs
 * excepted, FORMAT.md §5), tensor byte counts match their shapes, slabs are
 * 4096-aligned and large enough, metadata keys have their schema types, and the
 * canonical tensors of FORMAT.md §4.1 exist with their exact shapes. A malformed
 * file gives an error message, never an out-of-bounds read.
 */
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>

#include "hx_host.h"

namespace hx {

namespace {
constexpr uint32_t kMagic = 0x48545248u;   /* "HRTH" */
constexpr uint64_t kPreamble = 64, kTdirEntry = 128, kEdirEntry = 32;

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }
float rdf32(const uint8_t *p) { uint32_t u = rd32(p); float f; std::memcpy(&f, &u, 4); return f; }
bool inside(uint64_t off, uint64_t n, uint64_t size) { return off <= size && n <= size - off; }

std::string fmt(const char *f, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

/* metadata value types (FORMAT.md §3) */
enum { MT_U32 = 1, MT_F32 = 2, MT_U64 = 3, MT_STR = 4, MT_U32A = 5, MT_F32A = 6, MT_U8A = 7 };

struct MetaVal { int type; const uint8_t *p; uint32_t count; };

/* schema types of the keys this reader understands (FORMAT.md §3.1) */
const std::map<std::string, int> &schema() {
    static const std::map<std::string, int> s = {
        {"arch", MT_STR}, {"n_layers", MT_U32}, {"d_model", MT_U32}, {"vocab_size", MT_U32}, {"max_seq", MT_U32},
        {"norm_eps", MT_F32}, {"attn_kind", MT_U32}, {"n_heads", MT_U32}, {"n_kv_heads", MT_U32},
        {"head_dim", MT_U32}, {"qk_norm", MT_U32}, {"qkv_bias", MT_U32}, {"q_lora_rank", MT_U32},
        {"kv_lora_rank", MT_U32}, {"qk_nope_dim", MT_U32}, {"qk_rope_dim", MT_U32}, {"v_head_dim", MT_U32},
        {"rope_dim", MT_U32}, {"rope_style", MT_U32}, {"rope_attn_factor", MT_F32}, {"attn_scale", MT_F32},
        {"dense_ffn_dim", MT_U32}, {"n_experts", MT_U32}, {"top_k", MT_U32}, {"expert_ffn_dim", MT_U32},
        {"shared_ffn_dim", MT_U32}, {"shared_gate", MT_U32}, {"score_fn", MT_U32}, {"score_bias", MT_U32},
        {"n_group", MT_U32}, {"topk_group", MT_U32}, {"norm_topk_prob", MT_U32}, {"routed_scale", MT_F32},
        {"emb_scale", MT_F32}, {"residual_scale", MT_F32}, {"logit_scale", MT_F32}, {"tie_embeddings", MT_U32},
        {"layer_kind", MT_U8A}, {"bos_id", MT_U32}, {"eos_ids", MT_U32A}, {"tokenizer", MT_STR},
        {"chat_template", MT_STR}, {"source", MT_STR}, {"expert_dtype", MT_U32}};
    return s;
}

struct Meta {
    std::map<std::string, MetaVal> kv;
    bool has(const char *k) const { return kv.count(k) != 0; }
    bool u32(const char *k, uint32_t def, uint32_t lo, uint32_t hi, int &out, std::string &err) const {
        auto it = kv.find(k);
        const uint32_t v = it == kv.end() ? def : rd32(it->second.p);
        if (v < lo || v > hi) {
            err = fmt("metadata %s = %u out of range [%u, %u]%s", k, v, lo, hi, it == kv.end() ? " (default)" : "");
            return false;
        }
        out = (int)v;
        return true;
    }
    bool f32(const char *k, float def, float &out, std::string &err) const {
        auto it = kv.find(k);
        const float v = it == kv.end() ? def : rdf32(it->second.p);
        if (!std::isfinite(v)) { err = fmt("metadata %s is not finite", k); return false; }
        out = v;
        return true;
    }
};

bool parse_meta(const uint8_t *b, uint64_t n, Meta &m, std::string &err) {
    uint64_t p = 0;
    while (p < n) {
        if (n - p < 2) { err = "metadata entry truncated"; return false; }
        const uint32_t klen = rd16(b + p);
        p += 2;
        if (n - p < (uint64_t)klen + 1) { err = "metadata entry runs past the section"; return false; }
        std::string key((const char *)b + p, klen);
        p += klen;
        const int type = b[p++];
        uint64_t plen;
        uint32_t count = 0;
        if (type == MT_U32 || type == MT_F32) plen = 4;
        else if (type == MT_U64) plen = 8;
        else if (type >= MT_STR && type <= MT_U8A) {
            if (n - p < 4) { err = "metadata entry truncated"; return false; }
            count = rd32(b + p);
            p += 4;
            plen = (uint64_t)count * ((type == MT_STR || type == MT_U8A) ? 1u : 4u);
        } else {
            err = fmt("metadata '%.64s': unknown type %d", key.c_str(), type);
            return false;
        }
        if (n - p < plen) { err = fmt("metadata '%.64s' runs past the section", key.c_str()); return false; }
        auto s = schema().find(key);
        if (s != schema().end()) {
            if (s->second != type) { err = fmt("metadata '%s' has type %d, expected %d", key.c_str(), type, s->second); return false; }
            m.kv[key] = MetaVal{type, b + p, count};   /* later duplicates win */
        }
        p += plen;
    }
    return true;
}

bool build_config(const Meta &m, Config &c, std::string &err) {
    for (const char *k : {"n_layers", "d_model", "vocab_size", "n_heads"})
        if (!m.has(k)) { err = fmt("metadata is missing required key '%s'", k); return false; }
    const uint32_t BIG = 1u << 24;
#define U(k, def, lo, hi, dst) do { if (!m.u32(k, def, lo, hi, dst, err)) return false; } while (0)
#define F(k, def, dst) do { if (!m.f32(k, def, dst, err)) return false; } while (0)
    U("n_layers", 0, 1, 512, c.n_layers);
    U("d_model", 0, 1, 1u << 20, c.d_model);
    U("vocab_size", 0, 1, BIG, c.vocab);
    U("max_seq", 4096, 1, BIG, c.max_seq);
    F("norm_eps", 1e-6f, c.eps);
    if (c.eps < 0.0f) { err = "metadata norm_eps is negative"; return false; }
    U("attn_kind", 0, 0, 1, c.attn_kind);
    U("n_heads", 0, 1, 1u << 16, c.n_heads);
    U("n_kv_heads", (uint32_t)c.n_heads, 1, 1u << 16, c.n_kv_heads);
    U("head_dim", (uint32_t)(c.d_model / c.n_heads), 0, 1u << 16, c.head_dim);
    U("qk_norm", 0, 0, 2, c.qk_norm);
    U("qkv_bias", 0, 0, 1, c.qkv_bias);
    U("q_lora_rank", 0, 0, 1u << 20, c.q_lora);
    U("kv_lora_rank", 0, 0, 1u << 20, c.kv_lora);
    U("qk_nope_dim", 0, 0, 1u << 16, c.nope);
    U("qk_rope_dim", 0, 0, 1u << 16, c.rope_qk);
    U("v_head_dim", 0, 0, 1u << 16, c.v_head);
    const bool mla = c.attn_kind == ATTN_MLA;
    int qk_dim;
    if (mla) {
        if (c.kv_lora < 1 || c.v_head < 1 || c.nope + c.rope_qk < 1) { err = "MLA needs kv_lora_rank, v_head_dim, qk dims >= 1"; return false; }
        qk_dim = c.nope + c.rope_qk;
    } else {
        if (c.head_dim < 1) { err = "head_dim is 0"; return false; }
        if (c.n_heads % c.n_kv_heads) { err = fmt("n_heads %d is not a multiple of n_kv_heads %d", c.n_heads, c.n_kv_heads); return false; }
        qk_dim = c.head_dim;
    }
    const int rope_cap = mla ? c.rope_qk : c.head_dim;
    U("rope_dim", (uint32_t)rope_cap, 0, (uint32_t)rope_cap, c.rope_dim);
    if (c.rope_dim % 2) { err = fmt("rope_dim %d is odd", c.rope_dim); return false; }
    U("rope_style", 0, 0, 1, c.rope_style);
    F("rope_attn_factor", 1.0f, c.rope_factor);
    F("attn_scale", 1.0f / sqrtf((float)qk_dim), c.attn_scale);
    U("dense_ffn_dim", 0, 0, 1u << 20, c.dense_ffn);
    U("n_experts", 0, 0, 65536, c.n_experts);
    U("top_k", 0, 0, 65536, c.top_k);
    U("expert_ffn_dim", 0, 0, 1u << 20, c.expert_ffn);
    U("shared_ffn_dim", 0, 0, 1u << 20, c.shared_ffn);
    U("shared_gate", 0, 0, 1, c.shared_gate);
    U("score_fn", 0, 0, 1, c.score_fn);
    U("score_bias", 0, 0, 1, c.score_bias);
    U("n_group", 1, 1, 65536, c.n_group);
    U("topk_group", 1, 1, 65536, c.topk_group);
    U("norm_topk_prob", 0, 0, 1, c.norm_topk);
    F("routed_scale", 1.0f, c.routed_scale);
    F("emb_scale", 1.0f, c.emb_scale);
    F("residual_scale", 1.0f, c.resid_scale);
    F("logit_scale", 1.0f, c.logit_scale);
    U("tie_embeddings", 0, 0, 1, c.tie);
#undef U
#undef F
    c.layer_kind.assign((size_t)c.n_layers, c.n_experts > 0 ? 1 : 0);
    auto lk = m.kv.find("layer_kind");
    if (lk != m.kv.end()) {
        if (lk->second.count != (uint32_t)c.n_layers) { err = fmt("layer_kind has %u entries for %d layers", lk->second.count, c.n_layers); return false; }
        for (int i = 0; i < c.n_layers; i++) {
            if (lk->second.p[i] > 1) { err = fmt("layer_kind[%d] = %u", i, lk->second.p[i]); return false; }
            c.layer_kind[i] = lk->second.p[i];
        }
    }
    c.n_moe = 0;
    for (int i = 0; i < c.n_layers; i++) c.n_moe += c.layer_kind[i];
    if (c.n_moe > 0) {
        if (c.n_experts < 1) { err = "MoE layers but n_experts is 0"; return false; }
        if (c.top_k < 1 || c.top_k > c.n_experts) { err = fmt("top_k %d out of range [1, %d]", c.top_k, c.n_experts); return false; }
        if (c.expert_ffn < 1) { err = "MoE layers need expert_ffn_dim >= 1"; return false; }
        if (c.n_experts % c.n_group) { err = "n_experts is not a multiple of n_group"; return false; }
        if (c.topk_group > c.n_group) { err = "topk_group > n_group"; return false; }
        if ((int64_t)c.top_k > (int64_t)c.topk_group * (c.n_experts / c.n_group)) { err = "top_k exceeds the experts in topk_group groups"; return false; }
    } else {
        c.n_experts = c.top_k = c.shared_ffn = 0;
    }
    if (c.n_moe < c.n_layers && c.dense_ffn < 1) { err = "dense layers need dense_ffn_dim >= 1"; return false; }
    auto bos = m.kv.find("bos_id");
    const uint32_t b = bos == m.kv.end() ? 0xFFFFFFFFu : rd32(bos->second.p);
    if (b == 0xFFFFFFFFu) c.bos_id = -1;
    else if (b >= (uint32_t)c.vocab) { err = "bos_id >= vocab_size"; return false; }
    else c.bos_id = (int)b;
    auto eos = m.kv.find("eos_ids");
    if (eos != m.kv.end())
        for (uint32_t i = 0; i < eos->second.count; i++) {
            const uint32_t id = rd32(eos->second.p + 4 * (size_t)i);
            if (id >= (uint32_t)c.vocab) { err = "eos id >= vocab_size"; return false; }
            if (c.eos_ids.size() < 8) c.eos_ids.push_back((int)id);
        }
    auto arch = m.kv.find("arch");
    if (arch != m.kv.end()) c.arch.assign((const char *)arch->second.p, arch->second.count);
    return true;
}
} // namespace

uint64_t slab_layout(int dtype, int64_t D, int64_t F, uint64_t *og, uint64_t *ou, uint64_t *od) {
    const uint64_t rd = row_bytes(dtype, D), rf = row_bytes(dtype, F);
    if (!rd || !rf) { *og = *ou = *od = 0; return 0; }
    *og = 0;
    *ou = ((uint64_t)F * rd + 63) / 64 * 64;
    *od = (*ou + (uint64_t)F * rd + 63) / 64 * 64;
    return (*od + (uint64_t)D * rf + 4095) / 4096 * 4096;
}

ModelFile::~ModelFile() {
    if (map_) munmap(map_, size_);
}

const Tensor *ModelFile::tensor(const std::string &name) const {
    auto it = std::lower_bound(tensors.begin(), tensors.end(), name,
                               [](const Tensor &t, const std::string &n) { return t.name < n; });
    return it != tensors.end() && it->name == name ? &*it : nullptr;
}

const Tensor *ModelFile::layer_tensor(int layer, const char *suffix) const {
    return tensor("blk." + std::to_string(layer) + "." + suffix);
}

const ExpertEntry *ModelFile::expert(int layer, int e) const {
    if (experts.empty() || layer < 0 || layer >= cfg.n_layers || e < 0 || e >= cfg.n_experts) return nullptr;
    return &experts[(size_t)layer * cfg.n_experts + e];
}

bool ModelFile::open(const std::string &p, std::string &err) {
    path = p;
    const int fd = ::open(p.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) { err = fmt("cannot open %s", p.c_str()); return false; }
    struct stat st;
    if (fstat(fd, &st) != 0) { ::close(fd); err = "cannot stat the file"; return false; }
    size_ = (uint64_t)st.st_size;
    if (size_ < kPreamble) { ::close(fd); err = fmt("file too small (%llu bytes)", (unsigned long long)size_); return false; }
    void *mp = mmap(nullptr, size_, PROT_READ, MAP_SHARED, fd, 0);
    ::close(fd);
    if (mp == MAP_FAILED) { size_ = 0; err = "cannot map the file"; return false; }
    map_ = (uint8_t *)mp;
    const uint8_t *b = map_;
    if (rd32(b) != kMagic) { err = fmt("not a .hearth container (magic 0x%08x)", rd32(b)); return false; }
    if (rd32(b + 4) != 1) { err = fmt("unsupported format version %u", rd32(b + 4)); return false; }
    if (rd32(b + 56) != 4096) { err = "slab alignment must be 4096"; return false; }
    const uint64_t meta_off = rd64(b + 8), meta_bytes = rd64(b + 16), tdir = rd64(b + 24), n_t = rd64(b + 32);
    const uint64_t edir = rd64(b + 40), n_e = rd64(b + 48);
    if (!inside(meta_off, meta_bytes, size_)) { err = "metadata section lies outside the file"; return false; }
    if (n_t > size_ / kTdirEntry || !inside(tdir, n_t * kTdirEntry, size_)) { err = "tensor directory lies outside the file"; return false; }
    if (n_e > size_ / kEdirEntry || !inside(edir, n_e * kEdirEntry, size_)) { err = "expert directory lies outside the file"; return false; }
    Meta meta;
    if (!parse_meta(b + meta_off, meta_bytes, meta, err)) return false;
    if (!build_config(meta, cfg, err)) return false;
    const Config &c = cfg;
    const uint64_t want_e = c.n_moe ? (uint64_t)c.n_layers * (uint64_t)c.n_experts : 0;
    if (n_e != want_e) { err = fmt("%llu expert entries, expected %llu", (unsigned long long)n_e, (unsigned long long)want_e); return false; }

    struct Region { uint64_t lo, hi; std::string what; };
    std::vector<Region> regions = {{0, kPreamble, "preamble"}, {meta_off, meta_off + meta_bytes, "metadata"},
                                   {tdir, tdir + n_t * kTdirEntry, "tensor directory"},
                                   {edir, edir + n_e * kEdirEntry, "expert directory"}};
    tensors.resize(n_t);
    for (uint64_t i = 0; i < n_t; i++) {
        const uint8_t *e = b + tdir + kTdirEntry * i;
        const void *nul = std::memchr(e, 0, 80);
        if (!nul) { err = fmt("tensor entry %llu: name not NUL-terminated", (unsigned long long)i); return false; }
        Tensor &t = tensors[i];
        t.name.assign((const char *)e, (const char *)nul - (const char *)e);
        if (t.name.empty()) { err = "empty tensor name"; return false; }
        t.dtype = (int)rd32(e + 80);
        t.ndim = (int)rd32(e + 84);
        if (t.dtype < HEARTH_F32 || t.dtype > HEARTH_U8) { err = fmt("tensor '%s': unknown dtype %d", t.name.c_str(), t.dtype); return false; }
        if (t.ndim < 1 || t.ndim > 4) { err = fmt("tensor '%s': ndim %d", t.name.c_str(), t.ndim); return false; }
        uint64_t rows = 1;
        for (int k = 0; k < 4; k++) {
            const uint32_t d = rd32(e + 88 + 4 * k);
            if (k < t.ndim ? d < 1 : d != 1) { err = fmt("tensor '%s': bad shape entry %d", t.name.c_str(), k); return false; }
            t.shape[k] = d;
            if (k + 1 < t.ndim) rows *= d;
        }
        t.offset = rd64(e + 104);
        t.nbytes = rd64(e + 112);
        const size_t rb = row_bytes(t.dtype, t.shape[t.ndim - 1]);
        if (!rb || (rows > 0 && rb > UINT64_MAX / rows) || t.nbytes != rows * rb) {
            err = fmt("tensor '%s': nbytes does not match its shape and dtype", t.name.c_str());
            return false;
        }
        if (t.offset % 64) { err = fmt("tensor '%s': offset not 64-byte aligned", t.name.c_str()); return false; }
        if (!inside(t.offset, t.nbytes, size_)) { err = fmt("tensor '%s' lies outside the file", t.name.c_str()); return false; }
        regions.push_back({t.offset, t.offset + t.nbytes, "tensor '" + t.name + "'"});
    }
    std::sort(tensors.begin(), tensors.end(), [](const Tensor &x, const Tensor &y) { return x.name < y.name; });
    for (size_t i = 1; i < tensors.size(); i++)
        if (tensors[i].name == tensors[i - 1].name) { err = "duplicate tensor '" + tensors[i].name + "'"; return false; }

    experts.resize(n_e);
    std::map<uint64_t, std::pair<const ExpertEntry *, int>> slabs;   /* offset -> (entry, unaliased count) */
    for (uint64_t i = 0; i < n_e; i++) {
        const uint8_t *e = b + edir + kEdirEntry * i;
        ExpertEntry &x = experts[i];
        x.offset = rd64(e);
        x.nbytes = rd64(e + 8);
        x.dtype = rd32(e + 16);
        x.flags = rd32(e + 20);
        const int layer = (int)(i / (uint64_t)c.n_experts);
        if (x.offset % 4096 || x.nbytes % 4096) { err = fmt("expert entry %llu: offset/size not 4096-aligned", (unsigned long long)i); return false; }
        if (!inside(x.offset, x.nbytes, size_)) { err = fmt("expert entry %llu: slab outside the file", (unsigned long long)i); return false; }
        if (!c.layer_kind[layer]) {
            if (x.nbytes) { err = fmt("expert entry %llu: slab in dense layer %d", (unsigned long long)i, layer); return false; }
            continue;
        }
        if (!x.nbytes) { err = fmt("expert entry %llu: empty slab in MoE layer %d", (unsigned long long)i, layer); return false; }
        if (x.dtype > HEARTH_Q4) { err = fmt("expert entry %llu: bad slab dtype %u", (unsigned long long)i, x.dtype); return false; }
        uint64_t og, ou, od;
        const uint64_t need = slab_layout((int)x.dtype, c.d_model, c.expert_ffn, &og, &ou, &od);
        if (!need) { err = fmt("expert entry %llu: dims invalid for dtype %s", (unsigned long long)i, dtype_name((int)x.dtype)); return false; }
        if (x.nbytes < need) { err = fmt("expert entry %llu: slab of %llu bytes < %llu needed", (unsigned long long)i, (unsigned long long)x.nbytes, (unsigned long long)need); return false; }
        auto it = slabs.find(x.offset);
        if (it == slabs.end()) {
            slabs[x.offset] = {&x, (x.flags & 1u) ? 0 : 1};
        } else {
            if (it->second.first->nbytes != x.nbytes || it->second.first->dtype != x.dtype) {
                err = fmt("expert entries share offset %llu but differ in size or dtype", (unsigned long long)x.offset);
                return false;
            }
            it->second.second += (x.flags & 1u) ? 0 : 1;
            if (it->second.second > 1) { err = "two expert entries point at one slab without the aliased flag"; return false; }
        }
    }
    expert_region_bytes = slab_bytes_max = 0;
    for (auto &s : slabs) {
        regions.push_back({s.first, s.first + s.second.first->nbytes, "expert slab"});
        expert_region_bytes += s.second.first->nbytes;
        slab_bytes_max = std::max(slab_bytes_max, s.second.first->nbytes);
    }
    std::sort(regions.begin(), regions.end(), [](const Region &x, const Region &y) { return x.lo < y.lo; });
    for (size_t i = 1, m = 0; i < regions.size(); i++) {
        if (regions[i].lo < regions[m].hi) { err = regions[m].what + " overlaps " + regions[i].what; return false; }
        if (regions[i].hi > regions[m].hi) m = i;
    }

    /* canonical tensors (FORMAT.md §4.1) */
    auto need = [&](int layer, const char *suffix, int ndim, int64_t d0, int64_t d1, bool f32_only) -> bool {
        const std::string name = layer < 0 ? std::string(suffix) : "blk." + std::to_string(layer) + "." + suffix;
        const Tensor *t = tensor(name);
        if (!t) { err = "tensor '" + name + "' is missing"; return false; }
        if (t->ndim != ndim || t->shape[0] != d0 || (ndim == 2 && t->shape[1] != d1)) {
            err = fmt("tensor '%s' has shape [%lld, %lld] (ndim %d), expected [%lld, %lld]", name.c_str(),
                      (long long)t->shape[0], (long long)t->shape[1], t->ndim, (long long)d0, (long long)d1);
            return false;
        }
        if (f32_only && t->dtype != HEARTH_F32) { err = "tensor '" + name + "' must be F32"; return false; }
        if (t->dtype > HEARTH_Q4) { err = "tensor '" + name + "' has a dtype that is not a matrix dtype"; return false; }
        return true;
    };
#define NEED(...) do { if (!need(__VA_ARGS__)) return false; } while (0)
    const int64_t D = c.d_model, H = c.n_heads;
    NEED(-1, "tok_embd", 2, c.vocab, D, false);
    if (!c.tie) NEED(-1, "lm_head", 2, c.vocab, D, false);
    NEED(-1, "out_norm", 1, D, 1, true);
    if (c.rope_dim > 0) NEED(-1, "rope_inv_freq", 1, c.rope_dim / 2, 1, true);
    else if (tensor("rope_inv_freq")) { err = "rope_inv_freq present although rope_dim is 0"; return false; }
    for (int l = 0; l < c.n_layers; l++) {
        NEED(l, "attn_norm", 1, D, 1, true);
        NEED(l, "ffn_norm", 1, D, 1, true);
        if (c.attn_kind == ATTN_MLA) {
            if (c.q_lora > 0) {
                NEED(l, "attn_q_a", 2, c.q_lora, D, false);
                NEED(l, "attn_q_a_norm", 1, c.q_lora, 1, true);
                NEED(l, "attn_q_b", 2, H * (c.nope + c.rope_qk), c.q_lora, false);
            } else {
                NEED(l, "attn_q", 2, H * (c.nope + c.rope_qk), D, false);
            }
            NEED(l, "attn_kv_a", 2, c.kv_lora + c.rope_qk, D, false);
            NEED(l, "attn_kv_a_norm", 1, c.kv_lora, 1, true);
            NEED(l, "attn_kv_b", 2, H * (c.nope + c.v_head), c.kv_lora, false);
            NEED(l, "attn_o", 2, D, H * c.v_head, false);
        } else {
            const int64_t q = H * c.head_dim, kv = (int64_t)c.n_kv_heads * c.head_dim;
            NEED(l, "attn_q", 2, q, D, false);
            NEED(l, "attn_k", 2, kv, D, false);
            NEED(l, "attn_v", 2, kv, D, false);
            NEED(l, "attn_o", 2, D, q, false);
            if (c.qkv_bias) {
                NEED(l, "attn_q_bias", 1, q, 1, true);
                NEED(l, "attn_k_bias", 1, kv, 1, true);
                NEED(l, "attn_v_bias", 1, kv, 1, true);
            }
            if (c.qk_norm) {
                NEED(l, "attn_q_norm", 1, c.qk_norm == QKNORM_HEAD ? c.head_dim : q, 1, true);
                NEED(l, "attn_k_norm", 1, c.qk_norm == QKNORM_HEAD ? c.head_dim : kv, 1, true);
            }
        }
        if (!c.layer_kind[l]) {
            NEED(l, "ffn_gate", 2, c.dense_ffn, D, false);
            NEED(l, "ffn_up", 2, c.dense_ffn, D, false);
            NEED(l, "ffn_down", 2, D, c.dense_ffn, false);
            continue;
        }
        NEED(l, "moe_router", 2, c.n_experts, D, true);
        if (c.score_bias) NEED(l, "moe_router_bias", 1, c.n_experts, 1, true);
        if (c.shared_ffn > 0) {
            NEED(l, "shexp_gate", 2, c.shared_ffn, D, false);
            NEED(l, "shexp_up", 2, c.shared_ffn, D, false);
            NEED(l, "shexp_down", 2, D, c.shared_ffn, false);
            if (c.shared_gate) NEED(l, "shexp_gate_inp", 2, 1, D, false);
        }
    }
#undef NEED
    double dense = 0.0, emb = 0.0;
    dense_bytes = 0;
    for (const Tensor &t : tensors) {
        double el = 1.0;
        for (int k = 0; k < t.ndim; k++) el *= (double)t.shape[k];
        dense_bytes += t.nbytes;
        if (t.name == "rope_inv_freq") continue;
        dense += el;
        if (t.name == "tok_embd") emb = el;
    }
    const double per_expert = 3.0 * (double)c.d_model * (double)c.expert_ffn;
    params_total = dense + (c.n_moe ? (double)c.n_moe * c.n_experts * per_expert : 0.0);
    params_active = dense - (c.tie ? 0.0 : emb) + (c.n_moe ? (double)c.n_moe * c.top_k * per_expert : 0.0);
    return true;
}

/* ---- logging ---- */
static int g_log_level = LOG_WARN;
void set_log_level(int level) { g_log_level = level; }
int get_log_level() { return g_log_level; }
void log_msg(int level, const char *f, ...) {
    if (level > g_log_level) return;
    static const char *tag[] = {"error", "warn", "info", "debug"};
    char buf[1024];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    fprintf(stderr, "hearth[%s]: %s\n", tag[level < 0 ? 0 : level > 3 ? 3 : level], buf);
}

} // namespace hx
