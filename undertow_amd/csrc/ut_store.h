// ut_store.h -- the HBM tier of the expert store (host code).
//
// Routed experts that do not fit HBM live behind a byte-budgeted cache of
// expert slots in device memory, the device counterpart of undertow's
// DiskExpertStore + ExpertCache (undertow-io/src/store.rs:46-249,
// undertow-core/src/cache.rs:15-340).  A slot holds one expert's gate, up
// and down payloads and their scales in one block, so a miss is one
// host->device copy.  Misses are served from the converted checkpoint on
// disk (pread into pinned staging) or from a host memory pool.  Each MoE
// layer's device pointer table [6][E] names the slots of its cached experts
// (null for the others); the expert kernels read it as they read a resident
// table.  Results do not depend on the tier: the same bytes reach the same
// kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <list>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "ut_internal.h"
#include "ut_safetensors.h"

namespace ut {

struct StoreStats {
    // StoreStatsSnapshot (undertow-core/src/store.rs): hits, misses, bytes
    // read from the backing source, seconds spent reading, evictions, the
    // cache's bytes and budget, prefetch hints issued / dropped
    int64_t hits = 0, misses = 0, bytes_read = 0, evictions = 0;
    int64_t prefetch_issued = 0, prefetch_dropped = 0;
    double read_seconds = 0.0;
    int64_t bytes_used = 0, budget_bytes = 0, pinned = 0;
};

class ExpertStore {
public:
    enum Policy { LRU = 0, WEIGHTED = 1 };
    enum Source { DISK = 0, HOST_POOL = 1 };

    ~ExpertStore();

    // Shapes and format of every routed expert; budget in bytes; max_live:
    // experts one step may need at once (4 rows x top_k).
    int32_t init(ut_ctx *ctx, int64_t n_layers, int64_t E, int64_t H, int64_t I, int fmt,
                 int64_t budget_bytes, int policy, int64_t max_live);
    // The disk source: routed experts named as the converter writes them.
    int32_t attach_disk(const std::string &dir);
    // The host-pool source: pool_experts experts of slot layout in pinned
    // host memory; key (layer, e) reads pool entry (layer * E + e) % n.
    int32_t attach_host_pool(int64_t pool_experts, uint64_t seed, float std);
    // The device pointer table [6][E] of MoE layer `layer`.
    void set_table(int64_t layer, void **table_dev) { tables_[(size_t)layer] = table_dev; }

    // get_expert for every unique id of a step (TieredStore::get_expert,
    // store.rs:174-193): hits are touched, misses loaded into free or
    // evicted slots, the layer's table updated; all stream-ordered before
    // the step's expert launches.  ids [n] (host), -1 entries ignored.
    int32_t ensure(int64_t layer, const int32_t *ids, int64_t n);
    // pin_hottest (store.rs:146-166): loads and pins keys in order until
    // budget_bytes are pinned; out-of-range keys are skipped.
    int32_t pin(const int32_t *layer_expert, int64_t n, int64_t budget_bytes, int64_t *pinned);
    // Speculative loads for the keys a pilot routing predicts (prefetch,
    // store.rs:195-220): misses are loaded now if a slot is free of the
    // step's experts; the cost is counted as prefetch, not as misses.
    int32_t prefetch(int64_t layer, const int32_t *ids, int64_t n);

    const StoreStats &stats();
    // usage counts [n_layers][E] (TieredStore::usage)
    const std::vector<int64_t> &usage() const { return usage_; }
    int fmt() const { return fmt_; }
    int64_t slot_bytes() const { return slot_bytes_; }

private:
    struct Slot {
        int64_t key = -1;  // layer * E + expert, or -1 when free
        bool pinned = false;
        double score = 0.0;
        uint64_t last_tick = 0;
        std::list<int>::iterator lru_it;
    };
    int32_t load_into(int slot, int64_t layer, int64_t e);
    int32_t publish(int64_t layer);
    void touch(int slot);
    int victim(const std::unordered_set<int64_t> &keep);
    void evict(int slot);
    void enforce_budget(const std::unordered_set<int64_t> &keep);
    double effective(const Slot &s) const;
    void fill_pool(unsigned t, unsigned nt, int64_t pool_experts, uint64_t seed, float std, float qmax);

    ut_ctx *ctx_ = nullptr;
    int64_t L_ = 0, E_ = 0, H_ = 0, I_ = 0, capacity_ = 0;
    int fmt_ = 0, policy_ = LRU, source_ = DISK;
    int64_t off_[6] = {0, 0, 0, 0, 0, 0}, len_[6] = {0, 0, 0, 0, 0, 0};
    int64_t slot_bytes_ = 0;
    char *pool_ = nullptr;  // device slots
    std::vector<Slot> slots_;
    std::vector<int> free_;
    std::list<int> lru_;  // front = least recently used
    std::unordered_map<int64_t, int> where_;
    std::unordered_set<int64_t> step_keys_;  // the last ensure's experts (in flight)
    uint64_t tick_ = 0;
    double half_life_ = 512.0;
    std::vector<void **> tables_;
    std::vector<void *> mirror_;  // pinned host copies of the tables [n_layers][6][E]
    std::vector<char> dirty_;
    // sources
    st::Index idx_;
    std::vector<uint16_t> halves_;  // 16-bit scales before widening
    void *stage_[2] = {nullptr, nullptr};
    hipEvent_t stage_done_[2] = {nullptr, nullptr};
    bool stage_busy_[2] = {false, false};
    int stage_next_ = 0;
    char *host_pool_ = nullptr;
    int64_t host_pool_n_ = 0;
    std::vector<int64_t> usage_;
    StoreStats stats_;
};

}  // namespace ut
