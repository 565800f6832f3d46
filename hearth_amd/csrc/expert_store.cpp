/*
 * expert_store.cpp — the HBM expert cache (expert_store.h).
 */
#include "expert_store.h"

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <unordered_map>

namespace hx {

namespace {

constexpr uint64_t ALIGN = 256;
constexpr double HEAT_DECAY = 0.995;   /* per forward (reference default heat_decay, hx_store.h) */
constexpr double HOT_HEAT = 0.5 / (1.0 - HEAT_DECAY);   /* LFU: used in about half of all forwards */

uint64_t al(uint64_t x) { return (x + ALIGN - 1) / ALIGN * ALIGN; }

/* bytes of one tiled matrix (hx_device.h QMat layout) of the given dtype */
void qmat_bytes(int dtype, int rows, int cols, uint64_t &w, uint64_t &d) {
    const int rows_pad = (rows + 15) & ~15, nb = cols / 64, nbp = (nb + 1) & ~1;
    w = (uint64_t)(rows_pad / 16) * nbp * 1024 / (dtype == HEARTH_Q4 ? 2 : 1);
    d = 2ull * nbp * rows_pad;
}

double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

} // namespace

GpuExpertStore::~GpuExpertStore() {
    if (cs_) (void)hipStreamSynchronize(cs_);
    for (int i = 0; i < 2; i++) {
        if (pinned_[i]) (void)hipHostFree(pinned_[i]);
        if (dstage_[i]) (void)hipFree(dstage_[i]);
        if (staged_[i]) (void)hipEventDestroy(staged_[i]);
    }
    for (uint8_t *a : arena_) (void)hipHostFree(a);
    for (auto &pr : ev_pend_) ev_free_.insert(ev_free_.end(), {pr.first, pr.second});
    for (hipEvent_t ev : ev_free_) (void)hipEventDestroy(ev);
    if (htable_) (void)hipHostFree(htable_);
    if (done_) (void)hipEventDestroy(done_);
    if (pool_) (void)hipFree(pool_);
    if (cs_) (void)hipStreamDestroy(cs_);
}

hxd::QMat GpuExpertStore::carve(uint8_t *&p, int dtype, int rows, int cols) const {
    hxd::QMat m{};
    uint64_t wb, db;
    qmat_bytes(room_, rows, cols, wb, db);
    m.dtype = dtype;
    m.rows = rows;
    m.rows_pad = (rows + 15) & ~15;
    m.nb = cols / 64;
    m.nbp = (m.nb + 1) & ~1;
    m.w = p;
    p += al(wb);
    m.d = (const uint16_t *)p;
    p += al(db);
    return m;
}

int GpuExpertStore::room_dtype(const ModelFile &mf, int L, int E) {
    for (int l = 0; l < L; l++)
        for (int e = 0; e < E && mf.cfg.layer_kind[l]; e++)
            if (mf.expert(l, e)->dtype == HEARTH_Q8) return HEARTH_Q8;
    return HEARTH_Q4;
}

uint64_t GpuExpertStore::slot_bytes_for(int D, int F, int room) {
    uint64_t wg, dg, wd, dd;
    qmat_bytes(room, F, D, wg, dg);
    qmat_bytes(room, D, F, wd, dd);
    return 2 * (al(wg) + al(dg)) + al(wd) + al(dd);
}

bool GpuExpertStore::open(const ModelFile &mf, int L, int E, int D, int F, int n_slots, int policy, bool host_tier,
                          std::string &msg) {
    mf_ = &mf;
    L_ = L; E_ = E; D_ = D; F_ = F; n_slots_ = n_slots; policy_ = policy;
    if (const char *fl = std::getenv("HEARTH_GPU_STORE_FAIL_LOAD")) fail_load_ = std::atoll(fl);
    room_ = room_dtype(mf, L, E);
    slot_bytes_ = slot_bytes_for(D, F, room_);
    for (int l = 0; l < L; l++)
        for (int e = 0; e < E && mf.cfg.layer_kind[l]; e++) {
            const ExpertEntry *x = mf.expert(l, e);
            uint64_t og, ou, od;
            const uint64_t need = slab_layout((int)x->dtype, D, F, &og, &ou, &od);
            if (need > stage_bytes_) stage_bytes_ = need;
        }
    if (hipMalloc((void **)&pool_, slot_bytes_ * (uint64_t)n_slots) != hipSuccess) {
        msg = "out of device memory for the expert cache slots";
        return false;
    }
    if (hipStreamCreateWithFlags(&cs_, hipStreamNonBlocking) != hipSuccess || hipEventCreate(&done_) != hipSuccess ||
        hipHostMalloc((void **)&htable_, sizeof(hxd::ExpertW) * (size_t)E, hipHostMallocDefault) != hipSuccess) {
        msg = "HIP error creating the expert cache";
        return false;
    }
    std::memset(htable_, 0, sizeof(hxd::ExpertW) * (size_t)E);
    for (int i = 0; i < 2; i++)
        if (hipHostMalloc((void **)&pinned_[i], stage_bytes_, hipHostMallocDefault) != hipSuccess ||
            hipMalloc((void **)&dstage_[i], stage_bytes_) != hipSuccess || hipEventCreate(&staged_[i]) != hipSuccess) {
            msg = "out of memory for the expert cache staging";
            return false;
        }
    slot_.assign(n_slots, Slot{});
    uint8_t *p = pool_;
    for (int s = 0; s < n_slots; s++) {   /* slot s is [pool_ + s * slot_bytes_, + slot_bytes_) */
        slot_[s].w.gate = carve(p, room_, F, D);
        slot_[s].w.up = carve(p, room_, F, D);
        slot_[s].w.down = carve(p, room_, D, F);
    }
    slot_of_.assign((size_t)L * E, -1);
    heat_.assign((size_t)L * E, 0.0);
    busy_.assign(n_slots, 0);
    free_.clear();
    for (int s = n_slots - 1; s >= 0; s--) free_.push_back(s);
    if (host_tier) build_tier();
    return true;
}

/* Raw slab of expert key -> pinned staging buffer buf -> device staging -> repacked
 * into the slot matrices w on the copy stream; the caller records staged_[buf] after
 * its last use of the pair, which is free again once that event has passed. */
void GpuExpertStore::stage(int key, int buf, hxd::ExpertW &w) {
    const ExpertEntry *x = mf_->expert(key / E_, key % E_);
    const int dt = (int)x->dtype;
    uint64_t og, ou, od;
    const uint64_t len = std::min<uint64_t>(slab_layout(dt, D_, F_, &og, &ou, &od), x->nbytes);
    if (staged_used_[buf]) ck(hipEventSynchronize(staged_[buf]));
    std::memcpy(pinned_[buf], mf_->data(x->offset), len);
    ck(hipMemcpyAsync(dstage_[buf], pinned_[buf], len, hipMemcpyHostToDevice, cs_));
    w.gate.dtype = w.up.dtype = w.down.dtype = dt;
    hxl::repack(dstage_[buf] + og, 0, w.gate.rows_pad, w.gate, cs_);
    hxl::repack(dstage_[buf] + ou, 0, w.up.rows_pad, w.up, cs_);
    hxl::repack(dstage_[buf] + od, 0, w.down.rows_pad, w.down, cs_);
}

/* The pinned host tier: one slot image per physical slab, made by staging the slab
 * into a slot and copying the slot back (the device repack is the one layout code). */
void GpuExpertStore::build_tier() {
    std::unordered_map<uint64_t, int> phys;   /* file offset -> image index */
    std::vector<int> first;                   /* image index -> first key holding it */
    img_.assign((size_t)L_ * E_, nullptr);
    for (int l = 0; l < L_; l++)
        for (int e = 0; e < E_ && mf_->cfg.layer_kind[l]; e++)
            if (phys.emplace(mf_->expert(l, e)->offset, (int)first.size()).second) first.push_back(l * E_ + e);
    const uint64_t n_img = first.size();
    const uint64_t per = std::max<uint64_t>(1, (1ull << 30) / slot_bytes_);   /* images per pinned chunk */
    std::vector<uint8_t *> base(n_img);
    for (uint64_t i = 0; i < n_img; i += per) {
        const uint64_t n = std::min(per, n_img - i);
        uint8_t *a = nullptr;
        if (hipHostMalloc((void **)&a, n * slot_bytes_, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            for (uint8_t *x : arena_) (void)hipHostFree(x);
            arena_.clear();
            img_.clear();
            tier_bytes_ = 0;
            return;   /* loads stay staged */
        }
        arena_.push_back(a);
        for (uint64_t j = 0; j < n; j++) base[i + j] = a + j * slot_bytes_;
    }
    for (uint64_t i = 0; i < n_img; i++) {
        const int buf = (int)(i & 1), s = (int)(i % (uint64_t)n_slots_);
        uint8_t *sb = pool_ + (uint64_t)s * slot_bytes_;
        stage(first[i], buf, slot_[s].w);
        ck(hipMemcpyAsync(base[i], sb, slot_bytes_, hipMemcpyDeviceToHost, cs_));
        ck(hipEventRecord(staged_[buf], cs_));
        staged_used_[buf] = true;
    }
    ck(hipStreamSynchronize(cs_));
    for (int l = 0; l < L_; l++)
        for (int e = 0; e < E_ && mf_->cfg.layer_kind[l]; e++) img_[(size_t)l * E_ + e] = base[phys[mf_->expert(l, e)->offset]];
    tier_bytes_ = n_img * slot_bytes_;
    tier_ = true;
}

int GpuExpertStore::resident() const { return n_slots_ - (int)free_.size(); }

/* a is the better victim than b (store.c:166-177): unprotected first; LFU: lower
 * decayed heat; then least recently used; then the lower slot */
bool GpuExpertStore::cheaper(int a, int b) const {
    const Slot &x = slot_[a], &y = slot_[b];
    const bool px = protected_(x), py = protected_(y);
    if (px != py) return !px;
    if (policy_ == HEARTH_POLICY_LFU) {
        const double hx_ = heat_[x.key], hy = heat_[y.key];
        if (hx_ != hy) return hx_ < hy;
    }
    if (x.last_seq != y.last_seq) return x.last_seq < y.last_seq;
    return a < b;
}

/* Victim among the slots not serving the current layer (store.c:179-199): the
 * cheapest; -1 if none, or if only protected ones remain and allow_protected is 0. */
int GpuExpertStore::victim(bool allow_protected) {
    int best = -1;
    for (int s = 0; s < n_slots_; s++)
        if (!busy_[s] && (best < 0 || cheaper(s, best))) best = s;
    if (best >= 0 && !allow_protected && protected_(slot_[best])) return -1;
    return best;
}

void GpuExpertStore::evict(int s) {
    Slot &x = slot_[s];
    slot_of_[x.key] = -1;
    stats.evictions++;
    if (x.pf_unused) stats.prefetch_wasted++;
    x.pf_unused = false;
}

void GpuExpertStore::load(int key, int s) {
    if (fail_load_ > 0 && ++n_load_calls_ == fail_load_) throw DeviceError{hipErrorInvalidValue};
    hxd::ExpertW &w = slot_[s].w;
    uint8_t *sb = pool_ + (uint64_t)s * slot_bytes_;
    if (tier_) {   /* one copy of the slot image */
        const int dt = (int)mf_->expert(key / E_, key % E_)->dtype;
        w.gate.dtype = w.up.dtype = w.down.dtype = dt;
        ck(hipMemcpyAsync(sb, img_[key], slot_bytes_, hipMemcpyHostToDevice, cs_));
        stats.loads++;
        stats.bytes_read += slot_bytes_;
        return;
    }
    const int i = cur_;
    cur_ ^= 1;
    stage(key, i, w);
    ck(hipEventRecord(staged_[i], cs_));
    staged_used_[i] = true;
    const ExpertEntry *x = mf_->expert(key / E_, key % E_);
    uint64_t og, ou, od;
    stats.loads++;
    stats.bytes_read += std::min<uint64_t>(slab_layout((int)x->dtype, D_, F_, &og, &ou, &od), x->nbytes);
}

hipEvent_t GpuExpertStore::batch_ev() {
    if (ev_free_.empty()) {
        hipEvent_t ev;
        ck(hipEventCreate(&ev));
        return ev;
    }
    hipEvent_t ev = ev_free_.back();
    ev_free_.pop_back();
    return ev;
}

void GpuExpertStore::batch_begin() {
    harvest(false);
    hipEvent_t a = batch_ev(), b = batch_ev();
    ck(hipEventRecord(a, cs_));
    ev_pend_.emplace_back(a, b);
}

void GpuExpertStore::batch_end() { ck(hipEventRecord(ev_pend_.back().second, cs_)); }

void GpuExpertStore::harvest(bool wait) {
    while (!ev_pend_.empty()) {
        auto [a, b] = ev_pend_.front();
        if (wait) ck(hipEventSynchronize(b));
        else if (hipEventQuery(b) != hipSuccess) break;
        float ms = 0.0f;
        ck(hipEventElapsedTime(&ms, a, b));
        stats.copy_s += ms * 1e-3;
        ev_free_.push_back(a);
        ev_free_.push_back(b);
        ev_pend_.pop_front();
    }
}

void GpuExpertStore::ensure(int layer, const int *experts, int n, hxd::ExpertW *table_dev, hipStream_t compute) {
    const double t0 = now_s();
    const StoreStats st0 = stats;
    bool batch = false;
    int pend_key = -1, pend_slot = -1;   /* the miss whose load is being enqueued */
    std::fill(busy_.begin(), busy_.end(), 0);
    try {
        /* hits first, so that no miss of this layer evicts them */
        for (int j = 0; j < n; j++) {
            const int key = layer * E_ + experts[j], s = slot_of_[key];
            if (s >= 0) busy_[s] = 1;
        }
        for (int j = 0; j < n; j++) {
            const int e = experts[j], key = layer * E_ + e;
            int s = slot_of_[key];
            if (s >= 0) {
                stats.hits++;
                if (slot_[s].pf_unused) {
                    slot_[s].pf_unused = false;
                    stats.prefetch_used++;
                }
            } else {
                stats.misses++;
                if (!free_.empty()) {
                    s = free_.back();
                    free_.pop_back();
                } else {
                    s = victim(true);
                    evict(s);
                }
                slot_[s].key = key;
                slot_of_[key] = s;
                busy_[s] = 1;
                pend_key = key;
                pend_slot = s;
                if (!batch) batch_begin();
                batch = true;
                load(key, s);
                pend_key = pend_slot = -1;
            }
            slot_[s].prot_tick = 0;
            slot_[s].last_tick = now_;
            slot_[s].last_seq = ++seq_;
            heat_[key] += 1.0;
            htable_[e] = slot_[s].w;
        }
        if (batch) batch_end();
        ck(hipMemcpyAsync(table_dev, htable_, sizeof(hxd::ExpertW) * (size_t)E_, hipMemcpyHostToDevice, cs_));
        ck(hipEventRecord(done_, cs_));
        ck(hipStreamWaitEvent(compute, done_, 0));
    } catch (const DeviceError &) {
        /* the slot whose load did not enqueue holds no expert: unmap it, so that no later
         * call counts it as a hit */
        if (pend_key >= 0) unmap(pend_key, pend_slot);
        if (batch) (void)hipEventRecord(ev_pend_.back().second, cs_);   /* close the batch's event pair */
        stats = st0;
        throw;
    }
    stats.load_s += now_s() - t0;
}

void GpuExpertStore::prefetch(int layer, const int *experts, int n) {
    const double t0 = now_s();
    const StoreStats st0 = stats;
    bool batch = false;
    int pend_key = -1, pend_slot = -1;
    try {
        for (int j = 0; j < n; j++) {
            const int key = layer * E_ + experts[j];
            const int r = slot_of_[key];
            if (r >= 0) {   /* resident: keep it for the coming demand */
                slot_[r].prot_tick = now_ + 1;
                continue;
            }
            int s;
            if (!free_.empty()) {
                s = free_.back();
                free_.pop_back();
            } else {
                s = victim(false);
                if (s >= 0) {   /* never a hot expert (store.c:207-214) */
                    const Slot &v = slot_[s];
                    if (policy_ == HEARTH_POLICY_LFU ? heat_[v.key] >= HOT_HEAT : v.last_tick == now_) s = -1;
                }
                if (s < 0) {
                    stats.prefetch_dropped++;
                    continue;
                }
                evict(s);
            }
            Slot &x = slot_[s];
            x.key = key;
            x.pf_unused = true;
            x.prot_tick = now_ + 1;
            slot_of_[key] = s;
            pend_key = key;
            pend_slot = s;
            if (!batch) batch_begin();
            batch = true;
            load(key, s);
            pend_key = pend_slot = -1;
            stats.prefetch_issued++;
        }
        if (batch) batch_end();
    } catch (const DeviceError &) {
        if (pend_key >= 0) unmap(pend_key, pend_slot);
        if (batch) (void)hipEventRecord(ev_pend_.back().second, cs_);   /* close the batch's event pair */
        stats = st0;
        throw;
    }
    stats.load_s += now_s() - t0;
}

/* slot s, mapped to key but without its bytes: back to the free list */
void GpuExpertStore::unmap(int key, int s) {
    slot_of_[key] = -1;
    Slot &x = slot_[s];
    x.key = -1;
    x.pf_unused = false;
    x.prot_tick = 0;
    busy_[s] = 0;
    free_.push_back(s);
}

void GpuExpertStore::tick() {
    now_++;
    if (policy_ != HEARTH_POLICY_LFU) return;
    for (double &h : heat_) h *= HEAT_DECAY;
}

} // namespace hx
