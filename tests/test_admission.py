"""Host-side causal admission (vbm_admission_*, no GPU) against the reference's known answers, a
hand-worked trace and the Python restatement in oracle/admission.py."""
import ctypes as C
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "oracle"))
import admission as ref  # noqa: E402


# ------------------------------------------------------------------ helper known answers
# tests/test_moe_admission.cpp:12-45 of the reference, verbatim values.
COLDER = [
    ((0, 100, 99), (1, 0, 1), True), ((2, 0, 1), (1, 100, 99), False), ((0, 0, 99), (0, 100, 1), True),
    ((0, 100, 1), (0, 0, 99), False), ((2, 100, 1), (2, 0, 99), True), ((2, 0, 99), (2, 100, 1), False),
    ((0, 0, 1), (0, 0, 99), True), ((4, 10, 12), (4, 10, 12), False),
]


def test_helper_known_answers_library(vb):
    lib = vb.load()
    for cand, cur, expected in COLDER:
        assert lib.vbm_moe_colder_admission(*cand, *cur) == int(expected), (cand, cur)
    assert [lib.vbm_moe_probation_margin(o, h) for o, h in ((0, 0), (1, 0), (1, 1), (1, 2), (1, 3))] == [4, 7, 6, 5, 4]
    assert lib.vbm_moe_probation_margin(1, 2**64 - 1) == 4
    assert lib.vbm_moe_anchor_slots(100, 4, 80) == 24
    assert lib.vbm_moe_anchor_slots(100, 4, 10) == 10
    assert lib.vbm_moe_anchor_slots(100, 4, 0) == 0
    assert lib.vbm_moe_anchor_slots(4, 4, 0) == 0
    assert [lib.vbm_moe_cold_gpu_budget(c) for c in (0, 1, 2, 10, 128)] == [0, 0, 1, 1, 1]
    assert lib.vbm_moe_gpu_slot_limit(100, 0) == 100
    assert lib.vbm_moe_gpu_slot_limit(100, 1) == 101


def test_helper_known_answers_oracle():
    for cand, cur, expected in COLDER:
        assert ref.colder_admission(cand, cur) == expected
    assert [ref.probation_margin(o, h) for o, h in ((False, 0), (True, 0), (True, 1), (True, 2), (True, 3))] == [4, 7, 6, 5, 4]
    assert ref.probation_margin(True, 2**64 - 1) == 4
    assert [ref.anchor_slots(100, 4, s) for s in (80, 10, 0)] == [24, 10, 0] and ref.anchor_slots(4, 4, 0) == 0
    assert [ref.cold_gpu_budget(c) for c in (0, 1, 2, 10, 128)] == [0, 0, 1, 1, 1]
    assert ref.gpu_slot_limit(100, False) == 100 and ref.gpu_slot_limit(100, True) == 101


# ------------------------------------------------------------------ library wrapper
class LibAdmission:
    def __init__(self, vb, L, E, K, S, window=64, margin=4, policy=0):
        self.vb, self.K, self.E, self.L = vb, K, E, L
        h = C.c_void_p()
        vb.call("vbm_admission_create", L, E, K, S, window, margin, policy, C.byref(h))
        self.h = h.value

    def seed(self, layer, expert):
        s = C.c_int32()
        self.vb.call("vbm_admission_seed", self.h, layer, expert, C.byref(s))
        return s.value

    def admit(self, layer, selected):
        sel = np.ascontiguousarray(selected, np.int32)
        hits = np.zeros(self.K, np.int32)
        slots, experts, evicted = (np.zeros(self.K, np.int32) for _ in range(3))
        n = C.c_int64()
        self.vb.call("vbm_admission_admit", self.h, layer, sel.ctypes.data, hits.ctypes.data, slots.ctypes.data,
                     experts.ctypes.data, evicted.ctypes.data, C.byref(n))
        return hits.tolist(), [(int(slots[i]), int(experts[i]), int(evicted[i])) for i in range(n.value)]

    def slot_map(self, layer):
        m = np.zeros(self.E, np.int32)
        self.vb.call("vbm_admission_slot_map", self.h, layer, m.ctypes.data)
        return m.tolist()

    def stats(self):
        s = np.zeros(4, np.uint64)
        self.vb.call("vbm_admission_stats", self.h, s.ctypes.data)
        return [int(v) for v in s]

    def write_dispatch(self, layer, ids, weights, cold_rank=-1):
        ids = np.ascontiguousarray(ids, np.int32)
        w = np.ascontiguousarray(weights, np.float32)
        out = np.zeros((ids.shape[0], 4, self.K), np.float32)
        self.vb.call("vbm_admission_write_dispatch", self.h, layer, ids.ctypes.data, w.ctypes.data, ids.shape[0],
                     cold_rank, out.ctypes.data)
        return out

    def set_lfu(self, admit_after, fill_after):
        self.vb.call("vbm_admission_set_lfu", self.h, admit_after, fill_after)

    def lfu_state(self):
        counts = np.zeros(self.L * self.E, np.uint16)
        halvings = C.c_uint64()
        self.vb.call("vbm_admission_lfu_state", self.h, counts.ctypes.data, C.byref(halvings))
        return counts.tolist(), halvings.value

    def close(self):
        self.vb.call("vbm_admission_destroy", self.h)


# Worked by hand from llama-b11669-hybrid-experts.patch:3087-3242 (classic): one layer, 8 experts,
# top-2, 5 slots (0, 1 reserved), window 8 dispatches, margin 2.
HAND_TRACE = [
    ([0, 1], [0, 0], []),
    ([0, 2], [0, 0], [(2, 0, -1)]),            # first empty slot
    ([0, 1], [1, 0], [(3, 1, -1)]),            # slot 2 holds a selected expert: skipped
    ([2, 3], [0, 0], [(4, 2, -1)]),            # the empty slot beats occupied ones
    ([3, 5], [0, 0], []),                      # recent 2 < victim frequency 2 + margin 2
    ([3, 6], [0, 0], []),
    ([3, 7], [0, 0], [(3, 3, 1)]),             # recent 4 >= 2 + 2: evicts expert 1 (lowest recent)
    ([1, 2], [0, 1], []),                      # readmission needs 3 >= 3 + 2
    ([4, 5], [0, 0], []),                      # window slides: dispatch 1 leaves the history
]


@pytest.mark.parametrize("impl", ["library", "oracle"])
def test_hand_worked_classic_trace(vb, impl):
    a = LibAdmission(vb, 1, 8, 2, 5, window=8, margin=2) if impl == "library" else ref.Admission(1, 8, 2, 5, 8, 2)
    for selected, hits, made in HAND_TRACE:
        got_hits, got_made = a.admit(0, selected)
        assert (got_hits, got_made) == (hits, made), selected
    expected_map = [2, -1, 4, 3, -1, -1, -1, -1]
    got_map = a.slot_map(0) if impl == "library" else a.slot_map[:8]
    assert got_map == expected_map
    if impl == "library":
        assert a.stats() == [9, 2, 4, 1]
        a.close()


# Worked by hand from :3091-3137 (lfu): one layer, 8 experts, top-2, 5 slots, admit after 2
# demands, fill after 1. lfu_entries = 3, so the halving threshold is (2 + renewed / 20) x 3.
LFU_TRACE = [
    ([0, 1], [0, 0], [(2, 0, -1), (3, 1, -1)]),   # free slots fill after one demand
    ([2, 3], [0, 0], [(4, 2, -1)]),               # 3 would replace the LRU entry 0: count 1 < 2
    ([3, 0], [0, 1], [(3, 3, 1)]),                # count 2 >= 2 and the LRU victim (1) has count 1
    ([1, 5], [0, 0], []),                         # 8 demands >= 7.2: counts halve first
    ([5, 1], [0, 0], [(4, 1, 2)]),                # 1 (count 2) replaces 2 (count 0)
]


@pytest.mark.parametrize("impl", ["library", "oracle"])
def test_hand_worked_lfu_trace(vb, impl):
    if impl == "library":
        a = LibAdmission(vb, 1, 8, 2, 5, window=8, margin=4, policy=ref.LFU)
        a.set_lfu(2, 1)
    else:
        a = ref.Admission(1, 8, 2, 5, 8, 4, ref.LFU)
        a.lfu_admit_after, a.lfu_fill_after = 2, 1
    for selected, hits, made in LFU_TRACE:
        assert a.admit(0, selected) == (hits, made), selected
    got_map = a.slot_map(0) if impl == "library" else a.slot_map[:8]
    assert got_map == [2, 4, -1, 3, -1, -1, -1, -1]
    counts, halvings = a.lfu_state() if impl == "library" else (a.lfu_count, a.lfu_halvings)
    assert counts == [1, 2, 0, 1, 0, 1, 0, 0] and halvings == 1
    if impl == "library":
        assert a.stats() == [5, 1, 5, 2]
        a.close()


def _admissions_by_dispatch(a, seq):
    out = []
    for d, sel in enumerate(seq, 1):
        _, made = a.admit(0, sel)
        if made:
            out.append((d, made))
    return out


@pytest.mark.parametrize("impl", ["library", "oracle"])
def test_probation_delays_readmission_after_unreused_lifetime(vb, impl):
    """Top-1, one layer, 6 experts, 2 dynamic slots, window 8. Expert 0 is admitted at the 4th
    selection, evicted at dispatch 12 without a single hit while resident; its readmission then
    needs margin 4 + 3 = 7 recent selections (dispatch 19), where classic readmits at 16."""
    seq = [[0]] * 4 + [[1]] * 4 + [[2]] * 4 + [[0]] * 7
    expected = {ref.PROBATION: [(4, [(1, 0, -1)]), (8, [(2, 1, -1)]), (12, [(1, 2, 0)]), (19, [(2, 0, 1)])],
                ref.CLASSIC: [(4, [(1, 0, -1)]), (8, [(2, 1, -1)]), (12, [(1, 2, 0)]), (16, [(2, 0, 1)])]}
    for policy, want in expected.items():
        a = LibAdmission(vb, 1, 6, 1, 3, window=8, margin=4, policy=policy) if impl == "library" \
            else ref.Admission(1, 6, 1, 3, 8, 4, policy)
        assert _admissions_by_dispatch(a, seq) == want, policy
        if impl == "library":
            a.close()


@pytest.mark.parametrize("impl", ["library", "oracle"])
def test_anchored_floor_protects_the_first_seeds(vb, impl):
    """Ten slots, top-2, five seeded experts: anchor_slots(10, 2, 5) = 2 protects the seeds in slots
    2 and 3, so the first admissions evict the seeds in slots 4 and 5; classic evicts slots 2, 3."""
    for policy, evict in ((ref.ANCHORED, [(4, 6, 2), (5, 7, 3)]), (ref.CLASSIC, [(2, 6, 0), (3, 7, 1)])):
        a = LibAdmission(vb, 1, 8, 2, 10, window=8, margin=2, policy=policy) if impl == "library" \
            else ref.Admission(1, 8, 2, 10, 8, 2, policy)
        for e in range(5):
            a.seed(0, e)
        assert _admissions_by_dispatch(a, [[6, 7]] * 3) == [(2, evict)], policy
        if impl == "library":
            with pytest.raises(vb.VbmError):
                a.seed(0, 5)                              # seeding after a dispatch
            a.close()


def test_lfu_thresholds_are_validated(vb):
    a = LibAdmission(vb, 1, 8, 2, 5, policy=ref.LFU)
    for admit, fill in ((0, 1), (16, 1), (6, 0), (6, 16)):
        with pytest.raises(vb.VbmError):
            a.set_lfu(admit, fill)
    a.set_lfu(15, 15)
    a.close()
    b = LibAdmission(vb, 1, 8, 2, 10, policy=ref.ANCHORED)
    with pytest.raises(vb.VbmError):
        vb.call("vbm_admission_set_anchors", b.h, 1)      # anchored derives its floor from the seeds
    b.close()


def zipf_trace(rng, L, E, K, tokens, s=1.1, reuse=0.6):
    """Per layer a seeded permutation; Zipf(s) popularity; with p=reuse keep the previous set."""
    perms = [rng.permutation(E) for _ in range(L)]
    p = 1.0 / np.arange(1, E + 1) ** s
    p /= p.sum()
    prev = [None] * L
    out = []
    for _ in range(tokens):
        row = []
        for l in range(L):
            if prev[l] is not None and rng.random() < reuse:
                sel = prev[l]
            else:
                sel = [int(perms[l][i]) for i in rng.choice(E, K, replace=False, p=p)]
            prev[l] = sel
            row.append(sel)
        out.append(row)
    return out


@pytest.mark.parametrize("policy,margin", [(ref.CLASSIC, 4), (ref.LRU, 1), (ref.RANKED, 4), (ref.PROBATION, 4),
                                           (ref.ANCHORED, 4), (ref.LFU, 4)])
def test_library_matches_restatement_on_zipf_traces(vb, policy, margin):
    L, E, K, S = 4, 32, 4, 4 + 40
    rng = np.random.default_rng(policy + 5)
    lib, py = LibAdmission(vb, L, E, K, S, window=16, margin=margin, policy=policy), ref.Admission(L, E, K, S, 16, margin, policy)
    if policy == ref.LFU:                                 # thresholds that admit within a 200-token trace
        lib.set_lfu(3, 1)
        py.lfu_admit_after, py.lfu_fill_after = 3, 1
    for l in range(L):                                   # a frozen plan seeds a few experts per layer
        for e in range(3):
            assert lib.seed(l, (5 * l + 7 * e) % E) == py.seed(l, (5 * l + 7 * e) % E)
    for row in zipf_trace(rng, L, E, K, 200):
        for l, sel in enumerate(row):
            assert lib.admit(l, sel) == py.admit(l, sel)
    for l in range(L):
        assert lib.slot_map(l) == py.slot_map[l * E:(l + 1) * E]
    assert lib.stats() == [py.dispatch_calls, py.hits, py.admissions, py.evictions]
    assert py.admissions > 0 and (policy == ref.LRU or py.evictions > 0)
    if policy == ref.LFU:
        assert lib.lfu_state() == (py.lfu_count, py.lfu_halvings) and py.lfu_halvings > 0
    ids = np.array([[3, 9, 1, 30], [4, 5, 6, 7]])
    w = np.array([[0.4, 0.3, 0.2, 0.1], [0.25, 0.25, 0.25, 0.25]])
    for cold in (-1, 2):
        got = lib.write_dispatch(1, ids, w, cold)
        assert np.array_equal(got, np.array(py.write_dispatch(1, ids.tolist(), w.tolist(), cold), np.float32))
    lib.close()


def test_admission_rejects_bad_arguments(vb):
    h = C.c_void_p()
    with pytest.raises(vb.VbmError):
        vb.call("vbm_admission_create", 2, 8, 4, 4, 64, 4, 0, C.byref(h))      # no dynamic slot
    with pytest.raises(vb.VbmError):
        vb.call("vbm_admission_create", 2, 8, 4, 16, 4, 4, 0, C.byref(h))      # window < 8
    a = LibAdmission(vb, 2, 8, 2, 6)
    with pytest.raises(vb.VbmError):
        a.admit(0, [1, 9])                                                       # expert out of range
    a.admit(0, [1, 2])
    with pytest.raises(vb.VbmError):
        a.seed(1, 3)                                                             # seeding after a dispatch
    a.close()
