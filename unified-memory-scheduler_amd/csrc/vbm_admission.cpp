// Causal expert admission over one shared pool of expert slots (host-side control; no device
// calls). Restates llama_moe_cache's admission and dispatch bookkeeping:
//   admit          third_party/patches/llama-b11669-hybrid-experts.patch:3087-3242
//   write_dispatch llama-b11669-hybrid-experts.patch:3059-3084
//   helpers        llama-b11669-hybrid-experts.patch:3543-3574
//   frozen-plan seeding and the admission floor  llama-b11669-hybrid-experts.patch:2650-2695
// Policies (llama-b11669-hybrid-experts.patch:2375-2391): classic (recent-frequency margin), lru
// (free slot or least recently seen), ranked (classic with cold-start seed priority and recency
// tie-breaks), probation (classic whose margin grows after an admitted lifetime without reuse,
// :3116-3119), anchored (classic above a floor protecting up to a quarter of the dynamic slots
// for frozen-plan seeds, :2689-2691) and lfu (capped demand counts with periodic halving,
// :3092-3102, :3121-3137). Slots [0, n_used) are the reserved per-rank zero slots of misses;
// anchors follow them.
#include "vbm_internal.hpp"

#include <algorithm>
#include <cstdint>
#include <deque>
#include <memory>
#include <vector>

using namespace vbm;

struct vbm_admission {
    int64_t n_layers = 0, n_expert = 0, n_used = 0, n_slots = 0;
    int64_t admission_floor = 0;
    int64_t recent_window = 64;
    int32_t margin = 4;
    int policy = VBM_ADMIT_CLASSIC;
    uint64_t dispatch_calls = 0, pre_admission_hits = 0, admissions = 0, evictions = 0;
    int64_t next_seed_slot = 0;
    int32_t seeds = 0;
    std::vector<int32_t> key_of;        // [n_slots] key = layer * n_expert + expert, or -1
    std::vector<int32_t> slot_map;      // [n_layers][n_expert] slot or -1
    std::vector<int32_t> recent;        // [keys] selections inside the history window
    std::vector<uint64_t> last_seen;    // [keys] dispatch call of the last selection
    std::vector<int32_t> seed_priority; // [keys] frozen-plan order, 0 when not seeded
    std::deque<std::vector<int32_t>> history;
    bool floor_fixed = false;           // the floor (and LFU's entry count) is set at the first dispatch
    // lfu (:2188-2201)
    std::vector<uint16_t> lfu_count;    // [keys]
    uint64_t lfu_demands = 0, lfu_renewed = 0, lfu_entries = 0, lfu_halvings = 0;
    int lfu_admit_after = 6, lfu_fill_after = 1;
    // probation (:2214-2218): a key's last admitted lifetime
    struct Lifetime {
        uint64_t future_hits = 0;
        uint64_t bytes = 0;             // > 0 once the key was admitted dynamically
        bool dynamic = false;
    };
    std::vector<Lifetime> life;         // [keys]
};

constexpr uint16_t kLfuCap = 15;                 // :2196
constexpr int kLfuInsertsPerLayer = 4;           // :2201

namespace {

bool colder(int cf, int cs, uint64_t cl, int uf, int us, uint64_t ul) {
    if (cf != uf) return cf < uf;
    if (cf == 0 && cs != us) return cs < us;
    return cl < ul;
}

}  // namespace

extern "C" {

int vbm_moe_colder_admission(int candidate_frequency, int candidate_seed_priority, uint64_t candidate_last_seen,
                             int current_frequency, int current_seed_priority, uint64_t current_last_seen) {
    return colder(candidate_frequency, candidate_seed_priority, candidate_last_seen, current_frequency,
                  current_seed_priority, current_last_seen) ? 1 : 0;
}

int vbm_moe_probation_margin(int observed_lifetime, uint64_t future_hits) {
    return 4 + (observed_lifetime && future_hits < 3 ? 3 - static_cast<int>(future_hits) : 0);
}

int vbm_moe_anchor_slots(int capacity, int reserved, int seeds) {
    if (!(capacity >= reserved && seeds >= 0 && seeds <= capacity - reserved)) return -1;
    return std::min(seeds, (capacity - reserved) / 4);
}

int vbm_moe_cold_gpu_budget(int cold_experts) {
    if (cold_experts < 0) return -1;
    return cold_experts >= 2 ? 1 : 0;
}

int32_t vbm_moe_gpu_slot_limit(int32_t resident_slots, int cold_gpu) {
    if (!(resident_slots > 0 && resident_slots < INT32_MAX)) return -1;
    return resident_slots + (cold_gpu ? 1 : 0);
}

vbm_status vbm_admission_create(int64_t n_layers, int64_t n_expert, int64_t n_used, int64_t n_slots,
                                int64_t recent_window, int32_t margin, int policy, vbm_admission ** out) {
    return guarded([&] {
        require(out != nullptr, "null output");
        *out = nullptr;
        require(n_layers > 0 && n_expert > 0 && n_used > 0 && n_used <= n_expert, "invalid layer / expert shape");
        require(n_slots > n_used && n_slots < INT32_MAX, "the pool needs more slots than the reserved zero slots");
        require(n_layers * n_expert < INT32_MAX, "too many expert keys");
        require(recent_window >= 8 && recent_window <= 256, "recent window must be in 8..256");
        require(margin >= 1, "margin must be positive");
        require(policy >= VBM_ADMIT_CLASSIC && policy <= VBM_ADMIT_LFU, "unknown policy");
        auto a = std::make_unique<vbm_admission>();
        a->n_layers = n_layers;
        a->n_expert = n_expert;
        a->n_used = n_used;
        a->n_slots = n_slots;
        a->admission_floor = n_used;
        a->recent_window = recent_window;
        a->margin = margin;
        a->policy = policy;
        a->next_seed_slot = n_used;
        a->key_of.assign(static_cast<size_t>(n_slots), -1);
        a->slot_map.assign(static_cast<size_t>(n_layers * n_expert), -1);
        a->recent.assign(static_cast<size_t>(n_layers * n_expert), 0);
        a->last_seen.assign(static_cast<size_t>(n_layers * n_expert), 0);
        a->seed_priority.assign(static_cast<size_t>(n_layers * n_expert), 0);
        a->lfu_count.assign(static_cast<size_t>(n_layers * n_expert), 0);
        a->life.assign(static_cast<size_t>(n_layers * n_expert), vbm_admission::Lifetime{});
        *out = a.release();
    });
}

vbm_status vbm_admission_destroy(vbm_admission * a) {
    return guarded([&] { delete a; });
}

vbm_status vbm_admission_seed(vbm_admission * a, int64_t layer, int64_t expert, int32_t * slot) {
    return guarded([&] {
        require(a != nullptr, "null admission state");
        require(layer >= 0 && layer < a->n_layers && expert >= 0 && expert < a->n_expert, "seed out of range");
        require(a->dispatch_calls == 0, "seeding must precede the first dispatch");
        const int64_t key = layer * a->n_expert + expert;
        require(a->slot_map[key] < 0, "duplicate seed");
        require(a->next_seed_slot < a->n_slots, "seeds exceed the allocated expert slots");
        const int32_t s = static_cast<int32_t>(a->next_seed_slot++);
        a->slot_map[key] = s;
        a->key_of[s] = static_cast<int32_t>(key);
        ++a->seeds;
        a->seed_priority[key] = INT32_MAX - a->seeds;
        if (slot) *slot = s;
    });
}

vbm_status vbm_admission_set_anchors(vbm_admission * a, int32_t anchors) {
    return guarded([&] {
        require(a != nullptr, "null admission state");
        require(a->dispatch_calls == 0, "anchors must be set before the first dispatch");
        require(a->policy != VBM_ADMIT_ANCHORED, "the anchored policy derives its anchors from the seeds");
        require(anchors >= 0 && a->n_used + anchors < a->n_slots, "anchors exceed the pool");
        a->admission_floor = a->n_used + anchors;
    });
}

vbm_status vbm_admission_set_lfu(vbm_admission * a, int32_t admit_after, int32_t fill_after) {
    return guarded([&] {
        require(a != nullptr, "null admission state");
        require(admit_after >= 1 && admit_after <= kLfuCap, "LFU admission threshold must be in 1..15");   // :2403
        require(fill_after >= 1 && fill_after <= kLfuCap, "LFU fill threshold must be in 1..15");          // :2410
        a->lfu_admit_after = admit_after;
        a->lfu_fill_after = fill_after;
    });
}

vbm_status vbm_admission_admit(vbm_admission * a, int64_t layer, const int32_t * selected, int32_t * hits,
                               int32_t * admitted_slots, int32_t * admitted_experts, int32_t * evicted_keys,
                               int64_t * n_admitted) {
    return guarded([&] {
        require(a != nullptr && selected != nullptr && n_admitted != nullptr, "null argument");
        require(layer >= 0 && layer < a->n_layers, "layer out of range");
        const int64_t K = a->n_used, E = a->n_expert;
        std::vector<int32_t> keys(static_cast<size_t>(K));
        for (int64_t r = 0; r < K; ++r) {
            require(selected[r] >= 0 && selected[r] < E, "selected expert out of range");
            keys[r] = static_cast<int32_t>(layer * E + selected[r]);
        }
        const bool lru = a->policy == VBM_ADMIT_LRU, lfu = a->policy == VBM_ADMIT_LFU;
        const bool probation = a->policy == VBM_ADMIT_PROBATION;
        if (!a->floor_fixed) {   // :2686-2692, once the frozen plan's seeds are in place
            if (a->policy == VBM_ADMIT_ANCHORED)
                a->admission_floor = a->n_used + vbm_moe_anchor_slots(static_cast<int>(a->n_slots), static_cast<int>(a->n_used),
                                                                      static_cast<int>(a->next_seed_slot - a->n_used));
            a->lfu_entries = static_cast<uint64_t>(a->n_slots - a->admission_floor);
            a->floor_fixed = true;
        }
        ++a->dispatch_calls;
        if (a->policy == VBM_ADMIT_RANKED || lru || lfu)
            for (int32_t key : keys) a->last_seen[key] = a->dispatch_calls;
        if (lfu) {   // :3091-3102
            for (int32_t key : keys) a->lfu_count[key] += a->lfu_count[key] < kLfuCap;
            a->lfu_demands += static_cast<uint64_t>(K);
            a->lfu_renewed += static_cast<uint64_t>(K);
            const double entries = static_cast<double>(std::max<uint64_t>(a->lfu_entries, 1));
            const double window = std::min(5.0, 2.0 + 3.0 * static_cast<double>(a->lfu_renewed) / (20.0 * entries));
            if (static_cast<double>(a->lfu_demands) >= window * entries) {
                a->lfu_demands = 0;
                ++a->lfu_halvings;
                for (auto & c : a->lfu_count) c >>= 1;
            }
        }
        int lfu_inserts = 0;
        for (int64_t r = 0; r < K; ++r) {
            const bool hit = a->slot_map[keys[r]] >= 0;
            a->pre_admission_hits += hit;
            if (hits) hits[r] = hit ? 1 : 0;
            if (probation && hit && a->life[keys[r]].dynamic) ++a->life[keys[r]].future_hits;   // :3300-3305
        }
        a->history.push_back(keys);
        for (int32_t key : keys) ++a->recent[key];
        if (static_cast<int64_t>(a->history.size()) > a->recent_window * a->n_layers) {
            for (int32_t key : a->history.front()) --a->recent[key];
            a->history.pop_front();
        }
        int64_t n = 0;
        for (int64_t r = 0; r < K; ++r) {
            const int32_t key = keys[r];
            const vbm_admission::Lifetime & lk = a->life[key];
            const int margin = probation ? vbm_moe_probation_margin(lk.bytes > 0, lk.future_hits) : a->margin;
            if (a->slot_map[key] >= 0) continue;
            if (lfu ? (a->lfu_count[key] < std::min(a->lfu_fill_after, a->lfu_admit_after) || lfu_inserts >= kLfuInsertsPerLayer)
                    : a->recent[key] < margin)
                continue;
            int32_t victim_slot = -1;
            int victim_frequency = 0;
            if (lru || lfu) {
                uint64_t oldest = UINT64_MAX;
                for (int64_t slot = a->admission_floor; slot < a->n_slots; ++slot) {
                    const int32_t victim = a->key_of[slot];
                    if (victim < 0) { victim_slot = static_cast<int32_t>(slot); break; }
                    if (a->last_seen[victim] >= a->dispatch_calls) continue;   // selected by this dispatch
                    if (a->last_seen[victim] < oldest) { oldest = a->last_seen[victim]; victim_slot = static_cast<int32_t>(slot); }
                }
                if (lfu) {   // :3131-3137
                    if (victim_slot < 0) continue;
                    const int32_t victim = a->key_of[victim_slot];
                    if (a->lfu_count[key] < (victim < 0 ? a->lfu_fill_after : a->lfu_admit_after)) continue;
                    if (victim >= 0 && a->lfu_count[victim] >= a->lfu_count[key]) continue;
                    ++lfu_inserts;
                }
            } else {
                for (int64_t slot = a->admission_floor; slot < a->n_slots; ++slot) {
                    const int32_t victim = a->key_of[slot];
                    if (victim >= 0 && std::find(keys.begin(), keys.end(), victim) != keys.end()) continue;
                    const int frequency = victim >= 0 ? a->recent[victim] : 0;
                    bool prefer_tie = false;
                    if (a->policy == VBM_ADMIT_RANKED && victim_slot >= 0 && victim >= 0 && frequency == victim_frequency) {
                        const int32_t previous = a->key_of[victim_slot];
                        prefer_tie = colder(frequency, a->seed_priority[victim], a->last_seen[victim], victim_frequency,
                                            a->seed_priority[previous], a->last_seen[previous]);
                    }
                    if (victim_slot < 0 || frequency < victim_frequency || prefer_tie) {
                        victim_slot = static_cast<int32_t>(slot);
                        victim_frequency = frequency;
                        if (victim < 0) break;
                    }
                }
            }
            if (victim_slot < 0 || (!lru && !lfu && a->recent[key] < victim_frequency + margin)) continue;
            const int32_t victim = a->key_of[victim_slot];
            if (victim >= 0) {
                a->life[victim].dynamic = false;   // :3208-3216 (the lifetime's record stays)
                a->slot_map[victim] = -1;
                ++a->evictions;
            }
            a->key_of[victim_slot] = key;
            a->slot_map[key] = victim_slot;
            ++a->admissions;
            a->life[key] = vbm_admission::Lifetime{0, 1, true};   // :3229-3238 (only bytes > 0 is read)
            if (admitted_slots) admitted_slots[n] = victim_slot;
            if (admitted_experts) admitted_experts[n] = static_cast<int32_t>(key % E);
            if (evicted_keys) evicted_keys[n] = victim;
            ++n;
        }
        *n_admitted = n;
    });
}

vbm_status vbm_admission_write_dispatch(const vbm_admission * a, int64_t layer, const int32_t * ids, const float * weights,
                                        int64_t n_tokens, int32_t cold_rank, float * out) {
    return guarded([&] {
        require(a != nullptr && ids != nullptr && weights != nullptr && out != nullptr, "null argument");
        require(layer >= 0 && layer < a->n_layers && n_tokens > 0, "invalid dispatch shape");
        require(cold_rank < a->n_used, "cold rank out of range");
        const int64_t K = a->n_used, E = a->n_expert;
        for (int64_t t = 0; t < n_tokens; ++t)
            for (int64_t r = 0; r < K; ++r) {
                const int32_t expert = ids[t * K + r];
                require(expert >= 0 && expert < E, "expert id out of range");
                const int64_t slot = t == 0 && r == cold_rank ? a->n_slots : a->slot_map[layer * E + expert];
                const float w = weights[t * K + r];
                float * o = out + t * 4 * K;
                o[r] = slot >= 0 ? -1.0f : static_cast<float>(expert);
                o[K + r] = slot >= 0 ? static_cast<float>(slot) : static_cast<float>(r);
                o[2 * K + r] = slot >= 0 ? 0.0f : w;
                o[3 * K + r] = slot >= 0 ? 0.0f : 1.0f;
            }
    });
}

vbm_status vbm_admission_slot_map(const vbm_admission * a, int64_t layer, int32_t * map) {
    return guarded([&] {
        require(a != nullptr && map != nullptr && layer >= 0 && layer < a->n_layers, "invalid argument");
        std::copy_n(a->slot_map.begin() + layer * a->n_expert, a->n_expert, map);
    });
}

vbm_status vbm_admission_stats(const vbm_admission * a, uint64_t * stats) {
    return guarded([&] {
        require(a != nullptr && stats != nullptr, "invalid argument");
        stats[0] = a->dispatch_calls;
        stats[1] = a->pre_admission_hits;
        stats[2] = a->admissions;
        stats[3] = a->evictions;
    });
}

vbm_status vbm_admission_lfu_state(const vbm_admission * a, uint16_t * counts, uint64_t * halvings) {
    return guarded([&] {
        require(a != nullptr, "invalid argument");
        if (counts) std::copy(a->lfu_count.begin(), a->lfu_count.end(), counts);
        if (halvings) *halvings = a->lfu_halvings;
    });
}

}  // extern "C"
