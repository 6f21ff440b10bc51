"""Plain-Python restatement of llama_moe_cache's causal admission (TEST INFRASTRUCTURE ONLY).

Only tests/ may import this module, as the checker of the library's host-side admission state
(vbm_admission_*). It follows third_party/patches/llama-b11669-hybrid-experts.patch:
  admit            :3087-3242 (classic, lru, ranked, probation, anchored and lfu branches;
                   adaptive mode); policy switch :2375-2391, lfu state :2188-2201, lifetimes
                   :2214-2218 and :3300-3305, anchored floor :2686-2692
  write_dispatch   :3059-3084
  helpers          :3543-3574
  frozen-plan seed :2659-2680 (slots from n_expert_used upward, priority INT32_MAX - count)
"""
from __future__ import annotations

from collections import deque

INT32_MAX = 2**31 - 1
CLASSIC, LRU, RANKED, PROBATION, ANCHORED, LFU = 0, 1, 2, 3, 4, 5
LFU_CAP, LFU_INSERTS_PER_LAYER = 15, 4


def colder_admission(candidate, current) -> bool:
    """llama_moe_colder_admission (:3549-3555); ranks are (frequency, seed_priority, last_seen)."""
    cf, cs, cl = candidate
    uf, us, ul = current
    if cf != uf:
        return cf < uf
    if cf == 0 and cs != us:
        return cs < us
    return cl < ul


def probation_margin(observed_lifetime: bool, future_hits: int) -> int:
    """llama_moe_probation_margin (:3557-3559)."""
    return 4 + (3 - future_hits if observed_lifetime and future_hits < 3 else 0)


def anchor_slots(capacity: int, reserved: int, seeds: int) -> int:
    """llama_moe_anchor_slots (:3561-3564); -1 where the reference asserts."""
    if not (capacity >= reserved and 0 <= seeds <= capacity - reserved):
        return -1
    return min(seeds, (capacity - reserved) // 4)


def cold_gpu_budget(cold: int) -> int:
    """llama_moe_cold_gpu_budget (:3566-3569)."""
    return -1 if cold < 0 else (1 if cold >= 2 else 0)


def gpu_slot_limit(resident: int, cold_gpu: bool) -> int:
    """llama_moe_gpu_slot_limit (:3571-3574)."""
    if not (0 < resident < INT32_MAX):
        return -1
    return resident + (1 if cold_gpu else 0)


class Admission:
    """One shared slot pool for all routed layers (llama_moe_cache group state)."""

    def __init__(self, n_layers, n_expert, n_used, n_slots, recent_window=64, margin=4, policy=CLASSIC):
        self.L, self.E, self.K, self.S = n_layers, n_expert, n_used, n_slots
        self.floor = n_used
        self.window, self.margin, self.policy = recent_window, margin, policy
        self.dispatch_calls = self.hits = self.admissions = self.evictions = 0
        self.key_of = [-1] * n_slots
        self.slot_map = [-1] * (n_layers * n_expert)
        self.recent = [0] * (n_layers * n_expert)
        self.last_seen = [0] * (n_layers * n_expert)
        self.seed_priority = [0] * (n_layers * n_expert)
        self.history = deque()
        self.next_seed = n_used
        self.seeds = 0
        self.floor_fixed = False
        self.lfu_count = [0] * (n_layers * n_expert)
        self.lfu_demands = self.lfu_renewed = self.lfu_entries = self.lfu_halvings = 0
        self.lfu_admit_after, self.lfu_fill_after = 6, 1
        # lifetimes: [future_hits, bytes, dynamic]
        self.life = [[0, 0, False] for _ in range(n_layers * n_expert)]

    def seed(self, layer, expert):
        key = layer * self.E + expert
        slot = self.next_seed
        self.next_seed += 1
        self.slot_map[key] = slot
        self.key_of[slot] = key
        self.seeds += 1
        self.seed_priority[key] = INT32_MAX - self.seeds
        return slot

    def admit(self, layer, selected):
        """Returns (hits, [(slot, expert, evicted_key)])."""
        keys = [layer * self.E + e for e in selected]
        if not self.floor_fixed:
            if self.policy == ANCHORED:
                self.floor = self.K + anchor_slots(self.S, self.K, self.next_seed - self.K)
            self.lfu_entries = self.S - self.floor
            self.floor_fixed = True
        self.dispatch_calls += 1
        if self.policy in (LRU, RANKED, LFU):
            for k in keys:
                self.last_seen[k] = self.dispatch_calls
        if self.policy == LFU:
            for k in keys:
                self.lfu_count[k] += 1 if self.lfu_count[k] < LFU_CAP else 0
            self.lfu_demands += len(keys)
            self.lfu_renewed += len(keys)
            entries = float(max(self.lfu_entries, 1))
            window = min(5.0, 2.0 + 3.0 * self.lfu_renewed / (20.0 * entries))
            if self.lfu_demands >= window * entries:
                self.lfu_demands = 0
                self.lfu_halvings += 1
                self.lfu_count = [c >> 1 for c in self.lfu_count]
        lfu_inserts = 0
        hits = [1 if self.slot_map[k] >= 0 else 0 for k in keys]
        self.hits += sum(hits)
        if self.policy == PROBATION:
            for k, h in zip(keys, hits):
                if h and self.life[k][2]:
                    self.life[k][0] += 1
        self.history.append(keys)
        for k in keys:
            self.recent[k] += 1
        if len(self.history) > self.window * self.L:
            for k in self.history.popleft():
                self.recent[k] -= 1
        made = []
        for key in keys:
            margin = probation_margin(self.life[key][1] > 0, self.life[key][0]) if self.policy == PROBATION else self.margin
            if self.slot_map[key] >= 0:
                continue
            if self.policy == LFU:
                if self.lfu_count[key] < min(self.lfu_fill_after, self.lfu_admit_after) or lfu_inserts >= LFU_INSERTS_PER_LAYER:
                    continue
            elif self.recent[key] < margin:
                continue
            victim_slot, victim_frequency = -1, 0
            if self.policy in (LRU, LFU):
                oldest = None
                for slot in range(self.floor, self.S):
                    victim = self.key_of[slot]
                    if victim < 0:
                        victim_slot = slot
                        break
                    if self.last_seen[victim] >= self.dispatch_calls:
                        continue
                    if oldest is None or self.last_seen[victim] < oldest:
                        oldest, victim_slot = self.last_seen[victim], slot
                if self.policy == LFU:
                    if victim_slot < 0:
                        continue
                    victim = self.key_of[victim_slot]
                    if self.lfu_count[key] < (self.lfu_fill_after if victim < 0 else self.lfu_admit_after):
                        continue
                    if victim >= 0 and self.lfu_count[victim] >= self.lfu_count[key]:
                        continue
                    lfu_inserts += 1
            else:
                for slot in range(self.floor, self.S):
                    victim = self.key_of[slot]
                    if victim >= 0 and victim in keys:
                        continue
                    frequency = self.recent[victim] if victim >= 0 else 0
                    prefer_tie = False
                    if self.policy == RANKED and victim_slot >= 0 and victim >= 0 and frequency == victim_frequency:
                        prev = self.key_of[victim_slot]
                        prefer_tie = colder_admission((frequency, self.seed_priority[victim], self.last_seen[victim]),
                                                      (victim_frequency, self.seed_priority[prev], self.last_seen[prev]))
                    if victim_slot < 0 or frequency < victim_frequency or prefer_tie:
                        victim_slot, victim_frequency = slot, frequency
                        if victim < 0:
                            break
            if victim_slot < 0 or (self.policy not in (LRU, LFU) and self.recent[key] < victim_frequency + margin):
                continue
            victim = self.key_of[victim_slot]
            if victim >= 0:
                self.life[victim][2] = False
                self.slot_map[victim] = -1
                self.evictions += 1
            self.key_of[victim_slot] = key
            self.slot_map[key] = victim_slot
            self.admissions += 1
            self.life[key] = [0, 1, True]
            made.append((victim_slot, key % self.E, victim))
        return hits, made

    def write_dispatch(self, layer, ids, weights, cold_rank=-1):
        """[T][4][K] rows: (-1 or expert, slot or rank, 0 or weight, 0 or 1)."""
        out = []
        for t, (row_ids, row_w) in enumerate(zip(ids, weights)):
            cols = [[0.0] * self.K for _ in range(4)]
            for r, (e, w) in enumerate(zip(row_ids, row_w)):
                slot = self.S if (t == 0 and r == cold_rank) else self.slot_map[layer * self.E + e]
                cols[0][r] = -1.0 if slot >= 0 else float(e)
                cols[1][r] = float(slot) if slot >= 0 else float(r)
                cols[2][r] = 0.0 if slot >= 0 else float(w)
                cols[3][r] = 0.0 if slot >= 0 else 1.0
            out.append(cols)
        return out
