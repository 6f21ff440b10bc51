// Offline residency replay of decode routing traces: the explicit expert-cache cost models of the
// reference's trace analyzer, tools/benchmark/vrambridge-routing.py, for traces written by
// vbm_trace_* (or by the reference collector). Host-side; no device calls.
//
// Policies (vrambridge-routing.py:243-375, replay :441-512):
//   measured_static  the trace's static host/device placement, no uploads
//   train_static     the greedy byte-budget hot set of the training requests' counts (:232-240)
//   lru / lfu        demand admission after admit_after total references, at most capacity
//                    bytes; victims by last use (lru) or (count, last use) with no eviction of a
//                    more frequently used expert (lfu); uploads counted at layer end (:322-375)
//   belady_hits      hit-oriented, equal-size, end-of-layer admission with future knowledge
//   cost_aware       admission when a payback window of recent uses repays the upload and the
//                    benefit lost by the evicted experts (:269-320)
// and the latency model of Costs.latency (:212-223). Only the held-out (test) events are
// totalled; training events warm the cache (and their uploads are reported separately).
#include "vbm_internal.hpp"

#include <algorithm>
#include <cmath>
#include <deque>
#include <map>
#include <queue>
#include <set>
#include <unordered_map>
#include <vector>

using namespace vbm;

namespace {

using Key = std::pair<int32_t, int32_t>;   // (layer index in ascending id order, expert)

struct KeyHash {
    size_t operator()(const Key & k) const { return std::hash<int64_t>()((static_cast<int64_t>(k.first) << 32) ^ k.second); }
};

struct CostModel {
    double ram, pcie, gpu_us, sync_us;   // bytes per second; microseconds
    int passes;
    // (serial, optimistic, shared RAM bytes) of one layer's cold reads, GPU experts and uploads
    void latency(double cpu_bytes, double gpu_experts, double upload, double & serial, double & optimistic,
                 double & shared) const {
        const double gpu = gpu_experts * gpu_us / 1e6;
        const double sync = sync_us / 1e6;
        const double staging = passes * upload / ram;
        const double dma = std::max(upload / pcie, upload / ram);
        serial = cpu_bytes / ram + gpu + staging + dma + sync;
        shared = cpu_bytes + (passes + 1) * upload;
        optimistic = std::max(std::max(shared / ram, upload / pcie), gpu) + sync;
    }
};

struct Replay {
    const vbm_residency_layer * layers;
    int64_t n_layers;
    int policy;
    uint64_t capacity;
    int admit_after;
    CostModel cost;
    int64_t window_events;   // payback tokens x layers

    std::map<Key, uint64_t> resident;           // key -> clock of last use (ordered: key ties)
    std::unordered_map<Key, uint64_t, KeyHash> counts;
    uint64_t used = 0, clock = 0, rejected = 0;
    // cost-aware state
    std::unordered_map<Key, int64_t, KeyHash> recent;
    std::deque<std::pair<int64_t, std::vector<Key>>> history;
    // belady: per key, the event indices of its future uses
    std::map<Key, std::deque<int64_t>> future;

    uint64_t size_of(const Key & k) const { return layers[k.first].bytes_per_expert; }

    double benefit(const Key & k) const {
        const auto it = recent.find(k);
        const double r = it == recent.end() ? 0.0 : static_cast<double>(it->second);
        const double saved = static_cast<double>(size_of(k)) / cost.ram;
        const double extra = cost.gpu_us / 1e6;
        return r * std::max(0.0, saved - extra);
    }

    void cost_admit(const std::vector<Key> & keys, int64_t index, uint64_t & uploads, uint64_t & evictions) {
        history.emplace_back(index, keys);
        for (const Key & k : keys) ++recent[k];
        while (!history.empty() && history.front().first <= index - window_events) {
            for (const Key & k : history.front().second) {
                auto it = recent.find(k);
                if (--it->second <= 0) recent.erase(it);
            }
            history.pop_front();
        }
        std::map<Key, double> ben;
        for (const auto & kv : resident) ben[kv.first] = benefit(kv.first);
        for (const Key & k : keys) ben[k] = benefit(k);
        using Prio = std::pair<double, Key>;
        auto prio = [&](const Key & k) { return Prio{ben[k] / static_cast<double>(size_of(k)), k}; };
        std::priority_queue<Prio, std::vector<Prio>, std::greater<Prio>> order;   // lowest first
        for (const auto & kv : resident) order.push(prio(kv.first));
        std::set<Key> fresh;
        for (const Key & k : keys)
            if (!resident.count(k)) fresh.insert(k);
        std::vector<Key> cands(fresh.begin(), fresh.end());
        std::sort(cands.begin(), cands.end(), [&](const Key & a, const Key & b) {
            const double pa = prio(a).first, pb = prio(b).first;
            return pa != pb ? pa > pb : a < b;
        });
        for (const Key & k : cands) {
            const uint64_t size = size_of(k);
            const auto it = recent.find(k);
            const int64_t r = it == recent.end() ? 0 : it->second;
            if (r < admit_after || size > capacity) continue;
            uint64_t available = capacity - used;
            std::vector<Key> victims;
            double lost = 0.0;
            while (available < size && !order.empty()) {
                const Key v = order.top().second;
                order.pop();
                available += size_of(v);
                lost += ben[v];
                victims.push_back(v);
            }
            double serial, optimistic, shared;
            cost.latency(0.0, 0.0, static_cast<double>(size), serial, optimistic, shared);
            const double upload_seconds = serial - cost.sync_us / 1e6;
            if (available < size || ben[k] <= upload_seconds + lost) {
                for (const Key & v : victims) order.push(prio(v));
                ++rejected;
                continue;
            }
            for (const Key & v : victims) {
                resident.erase(v);
                used -= size_of(v);
            }
            resident[k] = clock;
            order.push(prio(k));
            used += size;
            uploads += size;
            evictions += victims.size();
        }
    }

    void demand_admit(const std::vector<Key> & keys) {
        const bool lfu = policy == VBM_RESIDENCY_LFU;
        for (const Key & k : keys) {
            const uint64_t size = size_of(k);
            if (resident.count(k) || counts[k] < static_cast<uint64_t>(admit_after) || size > capacity) continue;
            std::vector<Key> order;
            order.reserve(resident.size());
            for (const auto & kv : resident) order.push_back(kv.first);
            std::sort(order.begin(), order.end(), [&](const Key & a, const Key & b) {
                if (lfu && counts[a] != counts[b]) return counts[a] < counts[b];
                if (resident[a] != resident[b]) return resident[a] < resident[b];
                return a < b;
            });
            std::vector<Key> victims;
            uint64_t available = capacity - used;
            for (const Key & c : order) {
                if (available >= size) break;
                if (lfu && counts[c] > counts[k]) break;
                victims.push_back(c);
                available += size_of(c);
            }
            if (available < size) continue;
            for (const Key & v : victims) {
                resident.erase(v);
                used -= size_of(v);
            }
            resident[k] = clock;
            used += size;
        }
    }

    void belady(const std::vector<Key> & keys, int64_t index) {
        for (const Key & k : keys) {
            auto & q = future[k];
            require(!q.empty() && q.front() == index, "future-use queue is inconsistent");
            q.pop_front();
        }
        std::set<Key> cands;
        for (const auto & kv : resident) cands.insert(kv.first);
        for (const Key & k : keys) cands.insert(k);
        std::vector<std::pair<int64_t, Key>> live;
        for (const Key & k : cands) {
            const auto & q = future[k];
            if (!q.empty()) live.push_back({q.front(), k});
        }
        std::sort(live.begin(), live.end());
        const uint64_t size = layers[0].bytes_per_expert;
        const size_t keep = std::min<size_t>(live.size(), static_cast<size_t>(capacity / size));
        resident.clear();
        for (size_t i = 0; i < keep; ++i) resident[live[i].second] = clock;
        used = keep * size;
    }

    // One layer event; returns uploads and evictions (layer-end commit except cost-aware).
    void update(const std::vector<Key> & keys, int64_t index, uint64_t & uploads, uint64_t & evictions) {
        const std::map<Key, uint64_t> old = resident;
        ++clock;
        for (const Key & k : keys) {
            ++counts[k];
            auto it = resident.find(k);
            if (it != resident.end()) it->second = clock;
        }
        uploads = evictions = 0;
        if (policy == VBM_RESIDENCY_COST_AWARE) {
            cost_admit(keys, index, uploads, evictions);
        } else if (policy == VBM_RESIDENCY_BELADY_HITS) {
            belady(keys, index);
        } else {
            demand_admit(keys);
        }
        uint64_t check = 0;
        for (const auto & kv : resident) check += size_of(kv.first);
        require(used <= capacity && used == check, "cache byte-capacity invariant failed");
        if (policy == VBM_RESIDENCY_COST_AWARE) return;   // every admitted copy is charged
        for (const auto & kv : resident)
            if (!old.count(kv.first)) uploads += size_of(kv.first);
        for (const auto & kv : old)
            if (!resident.count(kv.first)) ++evictions;
    }
};

}  // namespace

extern "C" {

vbm_status vbm_residency_replay(const vbm_residency_layer * layers, int64_t n_layers, const int32_t * event_layer,
                                const int32_t * event_split, const int64_t * event_offsets, const int32_t * experts,
                                int64_t n_events, const vbm_residency_params * p, vbm_residency_totals * out) {
    return guarded([&] {
        require(layers && n_layers >= 1 && event_layer && event_split && event_offsets && experts && p && out,
                "null argument");
        require(n_events >= 0, "negative event count");
        require(p->policy >= VBM_RESIDENCY_MEASURED_STATIC && p->policy <= VBM_RESIDENCY_COST_AWARE,
                "Unknown residency policy");
        require(p->admit_after >= 1 && p->payback_tokens >= 1, "admission threshold and payback window must be >= 1");
        require(std::isfinite(p->ram_gbps) && p->ram_gbps > 0 && std::isfinite(p->pcie_gbps) && p->pcie_gbps > 0,
                "RAM and PCIe bandwidth must be finite and positive");
        require(std::isfinite(p->gpu_expert_us) && p->gpu_expert_us >= 0 && std::isfinite(p->layer_sync_us) &&
                    p->layer_sync_us >= 0, "GPU expert and layer-sync costs must be finite and nonnegative");
        require(p->staging_ram_passes == 0 || p->staging_ram_passes == 2, "staging RAM passes must be 0 or 2");
        for (int64_t l = 0; l < n_layers; ++l)
            require(layers[l].experts >= 1 && layers[l].bytes_per_expert >= 1 &&
                        layers[l].static_host_bytes_per_expert <= layers[l].bytes_per_expert,
                    "invalid layer description");
        *out = vbm_residency_totals{};
        Replay R;
        R.layers = layers;
        R.n_layers = n_layers;
        R.policy = p->policy;
        R.capacity = p->capacity_bytes;
        R.admit_after = p->admit_after;
        const CostModel cm{p->ram_gbps * 1e9, p->pcie_gbps * 1e9, p->gpu_expert_us, p->layer_sync_us,
                           p->staging_ram_passes};
        R.cost = cm;
        R.window_events = p->payback_tokens * n_layers;

        std::vector<std::vector<Key>> ev(static_cast<size_t>(n_events));
        for (int64_t i = 0; i < n_events; ++i) {
            const int32_t l = event_layer[i];
            require(l >= 0 && l < n_layers, "event layer out of range");
            for (int64_t j = event_offsets[i]; j < event_offsets[i + 1]; ++j) {
                require(experts[j] >= 0 && experts[j] < layers[l].experts, "expert id out of range");
                ev[static_cast<size_t>(i)].push_back({l, experts[j]});
            }
        }
        // train_static: the training hot set
        std::set<Key> fixed;
        if (p->policy == VBM_RESIDENCY_TRAIN_STATIC) {
            std::map<Key, uint64_t> freq;
            for (int64_t i = 0; i < n_events; ++i)
                if (event_split[i] == 0)
                    for (const Key & k : ev[static_cast<size_t>(i)]) ++freq[k];
            std::vector<Key> order;
            for (const auto & kv : freq) order.push_back(kv.first);
            std::sort(order.begin(), order.end(), [&](const Key & a, const Key & b) {
                if (freq[a] != freq[b]) return freq[a] > freq[b];
                if (R.size_of(a) != R.size_of(b)) return R.size_of(a) < R.size_of(b);
                return a < b;
            });
            uint64_t remaining = p->capacity_bytes;
            for (const Key & k : order)
                if (R.size_of(k) <= remaining) {
                    fixed.insert(k);
                    remaining -= R.size_of(k);
                }
        }
        if (p->policy == VBM_RESIDENCY_BELADY_HITS) {
            for (int64_t l = 1; l < n_layers; ++l)
                if (layers[l].bytes_per_expert != layers[0].bytes_per_expert) {
                    out->supported = 0;
                    return;
                }
            for (int64_t i = 0; i < n_events; ++i)
                for (const Key & k : ev[static_cast<size_t>(i)]) R.future[k].push_back(i);
        }
        out->supported = 1;
        bool testing = false;
        uint64_t warmup_rejected = 0;
        for (int64_t i = 0; i < n_events; ++i) {
            const auto & keys = ev[static_cast<size_t>(i)];
            const vbm_residency_layer & L = layers[event_layer[i]];
            const bool test = event_split[i] != 0;
            if (test && !testing) {
                if (p->cold_cache) {
                    R.resident.clear();
                    R.used = 0;
                }
                uint64_t initial = R.used;
                if (p->policy == VBM_RESIDENCY_MEASURED_STATIC) {
                    initial = p->static_device_expert_bytes;
                } else if (p->policy == VBM_RESIDENCY_TRAIN_STATIC) {
                    initial = 0;
                    for (const Key & k : fixed) initial += R.size_of(k);
                }
                out->initial_bytes = initial;
                warmup_rejected = R.rejected;
                testing = true;
            }
            uint64_t hits = 0, cold = 0, uploads = 0, evictions = 0;
            const uint64_t n = keys.size();
            if (p->policy == VBM_RESIDENCY_MEASURED_STATIC) {
                cold = n * L.static_host_bytes_per_expert;
                hits = L.static_host_bytes_per_expert == 0 ? n : 0;
            } else if (p->policy == VBM_RESIDENCY_TRAIN_STATIC) {
                for (const Key & k : keys) hits += fixed.count(k);
                cold = (n - hits) * L.bytes_per_expert;
            } else {
                for (const Key & k : keys) hits += R.resident.count(k);
                cold = (n - hits) * L.bytes_per_expert;
                R.update(keys, i, uploads, evictions);
            }
            if (!test) {
                out->warmup_upload_bytes += uploads;
                continue;
            }
            const uint64_t total = n * L.bytes_per_expert;
            double serial, optimistic, shared;
            cm.latency(static_cast<double>(cold), static_cast<double>(total - cold) / static_cast<double>(L.bytes_per_expert),
                       static_cast<double>(uploads), serial, optimistic, shared);
            out->expert_calls += n;
            out->full_hits += hits;
            out->bytes += total;
            out->cold_bytes += cold;
            out->upload_bytes += uploads;
            out->evictions += evictions;
            out->serial_s += serial;
            out->optimistic_s += optimistic;
            out->shared_ram_bytes += shared;
        }
        out->rejected = R.rejected - warmup_rejected;
        out->warmup_rejected = warmup_rejected;
    });
}

vbm_status vbm_residency_latency(const vbm_residency_params * p, double cpu_bytes, double gpu_experts, double upload_bytes,
                                 double * serial_s, double * optimistic_s, double * shared_ram_bytes) {
    return guarded([&] {
        require(p && serial_s && optimistic_s && shared_ram_bytes, "null argument");
        require(std::isfinite(p->ram_gbps) && p->ram_gbps > 0 && std::isfinite(p->pcie_gbps) && p->pcie_gbps > 0,
                "RAM and PCIe bandwidth must be finite and positive");
        require(p->staging_ram_passes == 0 || p->staging_ram_passes == 2, "staging RAM passes must be 0 or 2");
        const CostModel cm{p->ram_gbps * 1e9, p->pcie_gbps * 1e9, p->gpu_expert_us, p->layer_sync_us, p->staging_ram_passes};
        cm.latency(cpu_bytes, gpu_experts, upload_bytes, *serial_s, *optimistic_s, *shared_ram_bytes);
    });
}

}  // extern "C"
