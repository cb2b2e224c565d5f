// ut_store.hip -- the HBM tier of the expert store (host code): slots,
// LRU / weighted eviction, pinning, the disk and host-pool sources.
#include "ut_store.h"

#include <chrono>
#include <thread>
#include <cmath>
#include <cstring>

namespace ut {

namespace {

uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

int64_t align256(int64_t b) { return (b + 255) & ~int64_t(255); }

const char *kProj[3] = {"gate_proj", "up_proj", "down_proj"};

}  // namespace

ExpertStore::~ExpertStore() {
    if (ctx_) {
        (void)hipSetDevice(ctx_->device);
        (void)hipStreamSynchronize(ctx_->stream);
    }
    for (int i = 0; i < 2; i++) {
        if (stage_[i]) (void)hipHostFree(stage_[i]);
        if (stage_done_[i]) (void)hipEventDestroy(stage_done_[i]);
    }
    if (!mirror_.empty() && mirror_[0]) (void)hipHostFree(mirror_[0]);
    if (pool_) (void)hipFree(pool_);
    if (host_pool_) (void)hipHostFree(host_pool_);
}

int32_t ExpertStore::init(ut_ctx *ctx, int64_t n_layers, int64_t E, int64_t H, int64_t I, int fmt,
                          int64_t budget_bytes, int policy, int64_t max_live) {
    ctx_ = ctx;
    L_ = n_layers;
    E_ = E;
    H_ = H;
    I_ = I;
    fmt_ = fmt;
    policy_ = policy == WEIGHTED ? WEIGHTED : LRU;
    len_[0] = payload_bytes(fmt, I, H);
    len_[1] = len_[0];
    len_[2] = payload_bytes(fmt, H, I);
    len_[3] = fmt == UT_FMT_F32 ? 0 : I * 4;
    len_[4] = len_[3];
    len_[5] = fmt == UT_FMT_F32 ? 0 : H * 4;
    int64_t o = 0;
    for (int i = 0; i < 6; i++) {
        off_[i] = o;
        o += align256(len_[i]);
    }
    slot_bytes_ = o;
    capacity_ = budget_bytes > 0 ? budget_bytes / slot_bytes_ : 0;
    stats_.budget_bytes = budget_bytes;
    // a step may need max_live experts at once beyond what the budget retains
    const int64_t nslots = capacity_ + max_live;
    if (hipMalloc((void **)&pool_, (size_t)(nslots * slot_bytes_)) != hipSuccess) {
        (void)hipGetLastError();
        pool_ = nullptr;
        set_error(ctx, "expert cache: %lld slots of %lld bytes do not fit the device",
                  (long long)nslots, (long long)slot_bytes_);
        return UT_ERR_OOM;
    }
    slots_.assign((size_t)nslots, Slot{});
    for (int64_t i = nslots - 1; i >= 0; i--) free_.push_back((int)i);
    tables_.assign((size_t)L_, nullptr);
    void *mir = nullptr;
    const size_t tb = (size_t)E_ * 6 * sizeof(void *);
    if (hipHostMalloc(&mir, tb * (size_t)L_, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        set_error(ctx, "expert cache: pinned table mirror allocation failed");
        return UT_ERR_OOM;
    }
    memset(mir, 0, tb * (size_t)L_);
    mirror_.resize((size_t)L_);
    for (int64_t l = 0; l < L_; l++) mirror_[(size_t)l] = (char *)mir + (size_t)l * tb;
    dirty_.assign((size_t)L_, 0);
    usage_.assign((size_t)(L_ * E_), 0);
    return UT_OK;
}

int32_t ExpertStore::attach_disk(const std::string &dir) {
    std::string err;
    if (!st::open_dir(dir, idx_, err)) {
        set_error(ctx_, "%s", err.c_str());
        return err.find("No such file") != std::string::npos ? UT_ERR_IO : UT_ERR_FORMAT;
    }
    // every routed expert must be present with the store's format and shapes
    for (int64_t l = 0; l < L_; l++) {
        if (!tables_[(size_t)l]) continue;
        for (int64_t e = 0; e < E_; e++)
            for (int i = 0; i < 3; i++) {
                const std::string n = "model.layers." + std::to_string(l) + ".mlp.experts." +
                                      std::to_string(e) + "." + kProj[i] + ".weight";
                const st::Entry *p = idx_.find(n), *s = idx_.find(n + ".scales");
                if (!p) {
                    set_error(ctx_, "tensor not found: %s", n.c_str());
                    return UT_ERR_NOT_FOUND;
                }
                const int64_t out = i == 2 ? H_ : I_;
                // read_qtensor (reader.rs:410-430): a quantized payload is
                // taken raw by its byte count, its scales as f32 (F32, or
                // BF16 / F16 widened when loaded)
                const bool ok =
                    fmt_ == UT_FMT_F32
                        ? (p->dtype == st::ST_F32 && (int64_t)p->nbytes == len_[i])
                        : (s && s->shape.size() == 1 && s->shape[0] == out &&
                           (s->dtype == st::ST_F32 || s->dtype == st::ST_BF16 ||
                            s->dtype == st::ST_F16) &&
                           (int64_t)p->nbytes == len_[i]);
                if (!ok) {
                    set_error(ctx_, "%s: not a %s expert of [%lld, %lld] (all routed experts of a "
                                    "store share one format)",
                              n.c_str(), fmt_ == UT_FMT_INT4 ? "int4" : fmt_ == UT_FMT_INT8 ? "int8" : "f32",
                              (long long)out, (long long)(i == 2 ? I_ : H_));
                    return UT_ERR_FORMAT;
                }
            }
    }
    for (int i = 0; i < 2; i++) {
        if (hipHostMalloc(&stage_[i], (size_t)slot_bytes_, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&stage_done_[i], hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            set_error(ctx_, "expert cache: staging allocation failed");
            return UT_ERR_OOM;
        }
    }
    source_ = DISK;
    return UT_OK;
}

int32_t ExpertStore::attach_host_pool(int64_t pool_experts, uint64_t seed, float std) {
    if (pool_experts <= 0) return UT_ERR_ARG;
    const size_t bytes = (size_t)(pool_experts * slot_bytes_);
    if (hipHostMalloc((void **)&host_pool_, bytes, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        host_pool_ = nullptr;
        set_error(ctx_, "expert host pool of %zu bytes could not be pinned", bytes);
        return UT_ERR_OOM;
    }
    host_pool_n_ = pool_experts;
    // seeded experts: codes uniform over the format's range, per-row scales
    // |N(0, std)| / qmax (the synthetic benchmark's distributions); every
    // expert a pure function of (seed, index), filled by a few threads
    const float qmax = fmt_ == UT_FMT_INT4 ? 7.0f : 127.0f;
    unsigned nt = std::thread::hardware_concurrency();
    nt = nt < 1 ? 1 : (nt > 16 ? 16 : nt);
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < nt; t++)
        pool.emplace_back([this, t, nt, pool_experts, seed, std, qmax]() {
            fill_pool(t, nt, pool_experts, seed, std, qmax);
        });
    for (auto &th : pool) th.join();
    source_ = HOST_POOL;
    return UT_OK;
}

void ExpertStore::fill_pool(unsigned t, unsigned nt, int64_t pool_experts, uint64_t seed, float std,
                            float qmax) {
    for (int64_t x = t; x < pool_experts; x += nt) {
        char *base = host_pool_ + x * slot_bytes_;
        for (int i = 0; i < 3; i++) {
            uint64_t *w = (uint64_t *)(base + off_[i]);
            const int64_t words = (len_[i] + 7) / 8;
            uint64_t st = mix64(seed ^ mix64((uint64_t)(x * 8 + i)));
            for (int64_t k = 0; k < words; k++) {
                st += 0x9E3779B97F4A7C15ull;
                uint64_t v = mix64(st);
                if (fmt_ == UT_FMT_INT8) {
                    // bytes uniform in [-127, 127]
                    uint64_t r = 0;
                    for (int b = 0; b < 8; b++)
                        r |= (uint64_t)(uint8_t)(int8_t)((int)((v >> (8 * b)) & 0xFF) % 255 - 127) << (8 * b);
                    v = r;
                }
                w[k] = v;
            }
            float *sc = (float *)(base + off_[3 + i]);
            const int64_t rows = i == 2 ? H_ : I_;
            for (int64_t r = 0; r < rows; r++) {
                const uint64_t a = mix64(seed ^ mix64((uint64_t)(x * 8 + 3 + i) << 32 ^ (uint64_t)r));
                const float u1 = ((a >> 40) + 0.5f) * (1.0f / 16777216.0f);
                const float u2 = (((a >> 16) & 0xFFFFFF) + 0.5f) * (1.0f / 16777216.0f);
                sc[r] = fabsf(sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2)) * std / qmax;
            }
        }
    }
}

double ExpertStore::effective(const Slot &s) const {
    // WeightedExpertCache::effective (cache.rs): exponential decay of the
    // hit score with a half-life in ticks
    return s.score * std::pow(0.5, (double)(tick_ - s.last_tick) / half_life_);
}

void ExpertStore::touch(int slot) {
    Slot &s = slots_[(size_t)slot];
    if (s.pinned) return;
    if (policy_ == LRU) {
        lru_.erase(s.lru_it);
        lru_.push_back(slot);
        s.lru_it = std::prev(lru_.end());
    } else {
        s.score = effective(s) + 1.0;
        s.last_tick = tick_;
    }
}

int ExpertStore::victim(const std::unordered_set<int64_t> &keep) {
    if (policy_ == LRU) {
        for (int slot : lru_)
            if (!keep.count(slots_[(size_t)slot].key)) return slot;
        return -1;
    }
    int best = -1;
    double bs = 0.0;
    for (auto &kv : where_) {
        const Slot &s = slots_[(size_t)kv.second];
        if (s.pinned || keep.count(s.key)) continue;
        const double v = effective(s);
        if (best < 0 || v < bs) {
            best = kv.second;
            bs = v;
        }
    }
    return best;
}

void ExpertStore::evict(int slot) {
    Slot &s = slots_[(size_t)slot];
    const int64_t layer = s.key / E_, e = s.key % E_;
    void **mir = (void **)mirror_[(size_t)layer];
    for (int i = 0; i < 6; i++) mir[i * E_ + e] = nullptr;
    dirty_[(size_t)layer] = 1;
    where_.erase(s.key);
    if (!s.pinned && policy_ == LRU) lru_.erase(s.lru_it);
    s = Slot{};
    free_.push_back(slot);
    stats_.evictions++;
}

void ExpertStore::enforce_budget(const std::unordered_set<int64_t> &keep) {
    while ((int64_t)where_.size() > capacity_) {
        const int v = victim(keep);
        if (v < 0) break;
        evict(v);
    }
}

int32_t ExpertStore::load_into(int slot, int64_t layer, int64_t e) {
    char *dst = pool_ + (int64_t)slot * slot_bytes_;
    const auto t0 = std::chrono::steady_clock::now();
    if (source_ == HOST_POOL) {
        const int64_t x = (int64_t)((uint64_t)(layer * E_ + e) % (uint64_t)host_pool_n_);
        UT_CHECK_HIP(ctx_, hipMemcpyAsync(dst, host_pool_ + x * slot_bytes_, (size_t)slot_bytes_,
                                          hipMemcpyHostToDevice, ctx_->stream));
    } else {
        const int b = stage_next_;
        stage_next_ ^= 1;
        if (stage_busy_[b]) UT_CHECK_HIP(ctx_, hipEventSynchronize(stage_done_[b]));
        char *stg = (char *)stage_[b];
        for (int i = 0; i < 3; i++) {
            const std::string n = "model.layers." + std::to_string(layer) + ".mlp.experts." +
                                  std::to_string(e) + "." + kProj[i] + ".weight";
            const st::Entry *p = idx_.find(n);
            std::string err;
            if (!p || !st::read_at(idx_.shards[(size_t)p->shard], stg + off_[i], p->nbytes,
                                   p->offset, err)) {
                set_error(ctx_, "%s", p ? err.c_str() : ("tensor not found: " + n).c_str());
                return p ? UT_ERR_IO : UT_ERR_NOT_FOUND;
            }
            if (fmt_ != UT_FMT_F32) {
                const st::Entry *sc = idx_.find(n + ".scales");
                if (!sc || !st::read_f32_at(idx_.shards[(size_t)sc->shard], *sc,
                                            (float *)(stg + off_[3 + i]), halves_, err)) {
                    set_error(ctx_, "%s", sc ? err.c_str() : ("tensor not found: " + n + ".scales").c_str());
                    return sc ? UT_ERR_IO : UT_ERR_NOT_FOUND;
                }
            }
        }
        UT_CHECK_HIP(ctx_, hipMemcpyAsync(dst, stg, (size_t)slot_bytes_, hipMemcpyHostToDevice,
                                          ctx_->stream));
        UT_CHECK_HIP(ctx_, hipEventRecord(stage_done_[b], ctx_->stream));
        stage_busy_[b] = true;
    }
    stats_.read_seconds +=
        std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    stats_.bytes_read += len_[0] + len_[1] + len_[2] + len_[3] + len_[4] + len_[5];
    Slot &s = slots_[(size_t)slot];
    s.key = layer * E_ + e;
    s.pinned = false;
    s.score = 1.0;
    s.last_tick = tick_;
    if (policy_ == LRU) {
        lru_.push_back(slot);
        s.lru_it = std::prev(lru_.end());
    }
    where_[s.key] = slot;
    void **mir = (void **)mirror_[(size_t)layer];
    for (int i = 0; i < 6; i++) mir[i * E_ + e] = len_[i] ? dst + off_[i] : nullptr;
    dirty_[(size_t)layer] = 1;
    return UT_OK;
}

int32_t ExpertStore::publish(int64_t layer) {
    if (!dirty_[(size_t)layer] || !tables_[(size_t)layer]) return UT_OK;
    UT_CHECK_HIP(ctx_, hipMemcpyAsync(tables_[(size_t)layer], mirror_[(size_t)layer],
                                      (size_t)E_ * 6 * sizeof(void *), hipMemcpyHostToDevice,
                                      ctx_->stream));
    dirty_[(size_t)layer] = 0;
    return UT_OK;
}

int32_t ExpertStore::ensure(int64_t layer, const int32_t *ids, int64_t n) {
    if (layer < 0 || layer >= L_) return UT_ERR_ARG;
    std::unordered_set<int64_t> keep;
    std::vector<int64_t> order;
    for (int64_t j = 0; j < n; j++) {
        const int32_t e = ids[j];
        if (e < 0 || e >= E_) continue;  // the kernels report bad ids
        const int64_t key = layer * E_ + e;
        if (keep.insert(key).second) order.push_back(e);
    }
    for (int64_t e : order) {
        const int64_t key = layer * E_ + e;
        tick_++;
        usage_[(size_t)key]++;
        auto it = where_.find(key);
        if (it != where_.end()) {
            stats_.hits++;
            touch(it->second);
            continue;
        }
        stats_.misses++;
        int slot;
        if (!free_.empty()) {
            slot = free_.back();
            free_.pop_back();
        } else {
            slot = victim(keep);
            if (slot < 0) {
                set_error(ctx_, "expert cache: no slot free of the step's experts");
                return UT_ERR_STATE;
            }
            evict(slot);
            free_.pop_back();  // evict() returned it to the free list
        }
        UT_TRY(load_into(slot, layer, e));
    }
    enforce_budget(keep);
    step_keys_ = keep;
    return publish(layer);
}

int32_t ExpertStore::prefetch(int64_t layer, const int32_t *ids, int64_t n) {
    if (layer < 0 || layer >= L_) return UT_OK;
    // the last step's experts are about to run (their slots and its
    // published table must stay as they are): never a victim
    std::unordered_set<int64_t> keep = step_keys_;
    for (int64_t j = 0; j < n; j++) {
        const int32_t e = ids[j];
        if (e < 0 || e >= E_) continue;
        const int64_t key = layer * E_ + e;
        if (where_.count(key) || !keep.insert(key).second) continue;
        // only into a free slot or over a cold entry: a hint must not push
        // out the budget's working set beyond what an insert would
        int slot = -1;
        if (!free_.empty() && (int64_t)where_.size() < capacity_) {
            slot = free_.back();
            free_.pop_back();
        } else if ((int64_t)where_.size() >= capacity_ && capacity_ > 0) {
            slot = victim(keep);
            if (slot >= 0) {
                evict(slot);
                free_.pop_back();
            }
        }
        if (slot < 0) {
            stats_.prefetch_dropped++;
            continue;
        }
        tick_++;
        UT_TRY(load_into(slot, layer, e));
        stats_.prefetch_issued++;
    }
    return UT_OK;
}

int32_t ExpertStore::pin(const int32_t *le, int64_t n, int64_t budget_bytes, int64_t *pinned) {
    int64_t done = 0;
    // pins stay within the budget's slots; the step's transient slots stay free
    const int64_t max_pinned = capacity_;
    for (int64_t j = 0; j < n && done < budget_bytes; j++) {
        const int64_t layer = le[2 * j], e = le[2 * j + 1];
        if (layer < 0 || layer >= L_ || e < 0 || e >= E_ || !tables_[(size_t)layer]) continue;
        if (stats_.pinned >= max_pinned) break;
        const int64_t key = layer * E_ + e;
        auto it = where_.find(key);
        int slot;
        if (it != where_.end()) {
            slot = it->second;
            if (slots_[(size_t)slot].pinned) continue;
            if (policy_ == LRU) lru_.erase(slots_[(size_t)slot].lru_it);
        } else {
            if (!free_.empty()) {
                slot = free_.back();
                free_.pop_back();
            } else {
                slot = victim({});
                if (slot < 0) break;
                evict(slot);
                free_.pop_back();
            }
            UT_TRY(load_into(slot, layer, e));
            if (policy_ == LRU) lru_.erase(slots_[(size_t)slot].lru_it);
        }
        slots_[(size_t)slot].pinned = true;
        stats_.pinned++;
        done += slot_bytes_;
    }
    enforce_budget({});
    for (int64_t l = 0; l < L_; l++) UT_TRY(publish(l));
    UT_CHECK_HIP(ctx_, hipStreamSynchronize(ctx_->stream));
    if (pinned) *pinned = done;
    return UT_OK;
}

const StoreStats &ExpertStore::stats() {
    stats_.bytes_used = (int64_t)where_.size() * slot_bytes_;
    return stats_;
}

}  // namespace ut
