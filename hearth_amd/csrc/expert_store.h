/*
 * expert_store.h — the HBM expert cache: routed experts streamed from host memory into
 * a fixed pool of HBM slots when the experts do not fit (or HEARTH_GPU_EXPERT_CACHE_GB
 * sets a smaller budget). The reference's tiered store (engine/src/store.c, hx_store.h)
 * keeps slabs in a DRAM slot pool fed from NVMe; this is the same idea one tier up:
 *   - slot_of[layer * E + e] direct index, slot -> key back-map;
 *   - victims by LRU (least recently used) or LFU (decayed per-forward heat, ties by
 *     recency), store.c:166-214; slots of the layer being served are never victims;
 *   - a layer's demanded experts are made resident before its expert kernels run (the
 *     compute stream waits for the loads), so results never depend on the cache
 *     (weights are bytes, reference INV-DET-1);
 *   - the host tier: at open, every physical slab of the container (aliased entries
 *     share one) is repacked once into the slot layout (the MFMA tiles of its three
 *     matrices, exactly as a slot holds them) in pinned host memory, so that a load is
 *     a single hipMemcpyAsync of one slot image on the copy stream: no host copy, no
 *     repack, and back-to-back loads keep the host link busy. When the pinned tier
 *     cannot be allocated (or HEARTH_GPU_HOST_TIER=0), a load copies the slab from the
 *     mapped container into pinned staging, then to a device staging buffer, and
 *     repacks it there. The layer's device expert table gets the slot's matrices;
 *   - slots are sized for the widest expert dtype present (Q4-only models get Q4 slots);
 *   - prefetch (store.c:541-561, 207-214): experts predicted for the next MoE layer are
 *     loaded ahead into a free slot or an unprotected, not-hot victim (LRU: not used
 *     in this forward; LFU: heat below 0.5 / (1 - decay)); resident ones are
 *     protected for the current forward. A prefetched slot counts as used when it is
 *     first demanded and as wasted when it is evicted before that.
 * Every call comes from the engine's thread (an engine handle is single-threaded).
 */
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <deque>
#include <utility>
#include <vector>

#include "hx_host.h"
#include "hx_launch.h"

namespace hx {

/* A failed HIP call inside the engine or the store (caught at the C ABI). */
struct DeviceError {
    hipError_t e;
};

inline void ck(hipError_t e) {
    if (e != hipSuccess) throw DeviceError{e};
}

struct StoreStats {
    uint64_t hits = 0, misses = 0, evictions = 0, loads = 0, bytes_read = 0;
    uint64_t prefetch_issued = 0, prefetch_used = 0, prefetch_wasted = 0, prefetch_dropped = 0;
    double load_s = 0.0;   /* host time spent issuing loads and waiting for staging */
    double copy_s = 0.0;   /* copy-stream time of the load batches (HIP events; see harvest) */
};

class GpuExpertStore {
public:
    ~GpuExpertStore();
    /* n_slots >= E; policy HEARTH_POLICY_LRU / _LFU; host_tier: build the pinned slot
     * images (falls back to staged loads when the pinned memory cannot be had). Returns
     * false with msg on failure. */
    bool open(const ModelFile &mf, int L, int E, int D, int F, int n_slots, int policy, bool host_tier,
              std::string &msg);
    /* Makes experts[0..n) of layer resident, writes their matrices into table_dev (device
     * [E]) and makes `compute` wait for the loads. */
    void ensure(int layer, const int *experts, int n, hxd::ExpertW *table_dev, hipStream_t compute);
    /* Loads experts[0..n) of layer ahead of their demand where a slot can be had
     * without evicting a protected, in-use or hot expert; call after ensure() of the
     * current layer (its slots stay in use). */
    void prefetch(int layer, const int *experts, int n);
    /* forward boundary: LFU heat decay, protection expires */
    void tick();
    /* start of an API call that may run forwards: remembers the counters; rollback()
     * (after that call failed) puts them back, so a failed call leaves the statistics
     * as they were. Residency is not rolled back: every slot still mapped holds a load
     * that was enqueued in full. */
    void mark() { mark_ = stats; }
    void rollback() { stats = mark_; }
    /* the widest expert dtype of the container's MoE layers (Q8 if any expert is Q8) */
    static int room_dtype(const ModelFile &mf, int L, int E);
    /* HBM bytes of one slot for experts of D x F stored as `room` (Q8 or Q4) */
    static uint64_t slot_bytes_for(int D, int F, int room);
    int slots() const { return n_slots_; }
    int resident() const;
    /* adds the durations of the finished load batches to stats.copy_s; wait: all of them */
    void harvest(bool wait);
    uint64_t slot_bytes() const { return slot_bytes_; }
    bool host_tier() const { return tier_; }
    uint64_t host_tier_bytes() const { return tier_bytes_; }
    StoreStats stats;

private:
    StoreStats mark_;
    /* HEARTH_GPU_STORE_FAIL_LOAD=n at open: the n-th load since open fails once with a
     * HIP error before anything is enqueued (host-side test of the failure path) */
    long long fail_load_ = 0, n_load_calls_ = 0;
    struct Slot {
        int key = -1;
        uint64_t last_seq = 0;
        uint64_t last_tick = 0;   /* forward of the last demand */
        uint64_t prot_tick = 0;   /* protected while == now_ + 1 */
        bool pf_unused = false;   /* prefetched, not demanded yet */
        hxd::ExpertW w{};
    };
    const ModelFile *mf_ = nullptr;
    int L_ = 0, E_ = 0, D_ = 0, F_ = 0, n_slots_ = 0, policy_ = 0, room_ = HEARTH_Q8;
    uint64_t slot_bytes_ = 0, stage_bytes_ = 0, seq_ = 0, now_ = 0;
    uint8_t *pool_ = nullptr;
    std::vector<Slot> slot_;
    std::vector<int> slot_of_, free_;
    std::vector<double> heat_;
    std::vector<uint8_t> busy_;       /* slot holds an expert of the layer being served */
    hipStream_t cs_ = nullptr;        /* copy stream (default priority) */
    uint8_t *pinned_[2] = {nullptr, nullptr}, *dstage_[2] = {nullptr, nullptr};
    hipEvent_t staged_[2] = {nullptr, nullptr};
    bool staged_used_[2] = {false, false};
    int cur_ = 0;
    hxd::ExpertW *htable_ = nullptr;  /* pinned [E]: entries written this call */
    hipEvent_t done_ = nullptr;
    bool tier_ = false;               /* loads come from the pinned slot images */
    uint64_t tier_bytes_ = 0;
    std::vector<uint8_t *> arena_;    /* pinned chunks holding the slot images */
    std::vector<const uint8_t *> img_;   /* [L * E]: slot image of each expert (MoE layers) */
    void build_tier();
    /* event pairs bracketing the loads of one ensure() or prefetch() call on cs_ */
    std::vector<hipEvent_t> ev_free_;
    std::deque<std::pair<hipEvent_t, hipEvent_t>> ev_pend_;
    hipEvent_t batch_ev();
    void batch_begin();
    void batch_end();
    void stage(int key, int buf, hxd::ExpertW &w);
    hxd::QMat carve(uint8_t *&p, int dtype, int rows, int cols) const;
    bool protected_(const Slot &x) const { return x.prot_tick == now_ + 1; }
    bool cheaper(int a, int b) const;
    int victim(bool allow_protected);
    void evict(int s);
    void unmap(int key, int s);
    void load(int key, int slot);
};

} // namespace hx
