"""CPU: pins oracle/cache_model.py (the cache state machine oracle) with
scenarios worked out by hand from kernels/moe-cache.cu:525-775, invariants
checked over random traces, and the reference's seed file fixture."""
from pathlib import Path

import numpy as np
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle.cache_model import MISS_CAP, CacheModel, parse_seed_file, parse_seed_text

FIXTURE = Path(__file__).resolve().parent / "golden" / "moe_seed.txt"


def test_seed_fixture_shape():
    """assets/moe_seed.txt of the reference: 144 tensors (48 layers x gate/up/down), 167-364 ids per line."""
    seed = parse_seed_file(FIXTURE)
    assert len(seed) == 144
    names = {f"blk.{l}.ffn_{m}_exps.weight" for l in range(48) for m in ("gate", "up", "down")}
    assert set(seed) == names
    lens = [len(v) for v in seed.values()]
    assert min(lens) == 167 and max(lens) == 364
    assert seed["blk.47.ffn_gate_exps.weight"][:3] == [333, 183, 357]
    for v in seed.values():
        assert len(set(v)) == len(v) and all(0 <= e < 512 for e in v)   # a frequency ordering: distinct ids


def test_seed_parser_strtol_edge_cases():
    s = parse_seed_text("a 1,2,3\nb\nc 7,,8\nd -5,4x,9\ne  12\na 9\n" + "f " + ",".join(map(str, range(5))) + "\n")
    assert s["a"] == [9]                 # a later line replaces an earlier one
    assert "b" not in s                  # no space: skipped
    assert s["c"] == [7]                 # an empty field stops the line
    assert s["d"] == [-5, 4]             # parsing stops at the first non-number ("x")
    assert s["e"] == [12]                # leading blanks are skipped by strtol
    assert s["f"] == [0, 1, 2, 3, 4]


def test_registration_budget_and_seed_by_hand():
    eb = 100
    m = CacheModel(slots=4, budget_bytes=10 * eb, margin_bytes=0, seed={"t0": [3, 3, 99, 1, -1, 2, 0, 5]})
    e0 = m.register("p0", "t0", 8, eb, free_bytes=1000 * eb)
    assert e0.n_slots == 4
    assert e0.expert_of == [3, 1, 2, 0]          # repeated 3, out-of-range 99 and -1 skipped; stops at 4
    e1 = m.register("p1", "t1", 8, eb, free_bytes=1000 * eb)
    assert e1.n_slots == 4 and e1.expert_of == [-1] * 4
    e2 = m.register("p2", "t2", 8, eb, free_bytes=1000 * eb)
    assert e2.n_slots == 2                        # budget 10 slots, 8 used
    e3 = m.register("p3", "t3", 8, eb, free_bytes=3 * eb)
    assert e3.n_slots == 0                        # budget exhausted (and free memory binds too)
    assert m.register("p0", "other", 8, eb, free_bytes=0) is e0   # keyed by data pointer


def test_second_sighting_admission_and_lru_by_hand():
    m = CacheModel(slots=2, margin_bytes=0)
    e = m.register("p", "t", 6, 1, free_bytes=1 << 40)
    m.record(e, None, [[1, 2]])                   # misses: 1, 2 (first sightings)
    assert m.count == 2 and m.log[:2] == [1, 2] and m.hits == 0
    m.step()                                      # no promotion on first sighting
    assert e.expert_of == [-1, -1] and m.clock == 1
    m.record(e, None, [[1, 3]])                   # 1 second sighting -> slot 0; 3 first
    m.step()
    assert e.expert_of == [1, -1] and e.slot_of[1] == 0
    m.record(e, None, [[1, 2]])                   # 1 hit (stamp 2); 2 second sighting -> slot 1
    assert m.hits == 1
    m.step()
    assert e.expert_of == [1, 2]
    m.record(e, None, [[3, 1]])                   # 3: 2nd sighting, pool full -> evict min stamp
    # stamps: expert 1 stamped at clock 3 now, expert 2 stamped at clock 2 -> victim slot 1
    m.step()
    assert e.expert_of == [1, 3] and e.slot_of[2] == -1 and m.evictions == 1


def test_eviction_ties_take_lowest_slot_and_stamp_mirror_is_per_step():
    m = CacheModel(slots=2, margin_bytes=0, seed={"t": [0, 1]})
    e = m.register("p", "t", 8, 1, free_bytes=1 << 40)
    assert e.expert_of == [0, 1]
    m.record(e, None, [[5, 6]])
    m.step()
    m.record(e, None, [[5, 6]])                   # both reach 2 sightings in one step
    m.step()
    # stamps of residents 0 and 1 are both 0 -> slot 0 evicted first (strict <); the mirror is then
    # stale for the rest of the step: the just-promoted 5 carries mirror stamp 1 (its miss at clock 1),
    # resident 1 still 0 -> slot 1 evicted for 6
    assert e.expert_of == [5, 6] and m.evictions == 2


def test_promotion_cap_and_miss_log_overflow():
    m = CacheModel(slots=100, margin_bytes=0, max_promotions=3)
    e = m.register("p", "t", 100, 1, free_bytes=1 << 40)
    ids = [[i] for i in range(10)]
    m.record(e, None, ids)
    m.record(e, None, ids)                        # every expert twice in one step
    m.step()
    assert m.promotions == 3                      # scan stops after the cap
    # log = [0..9, 0..9]: the first pass counts every expert once, the second pass promotes 0, 1, 2
    # (their counts reset to 0) and stops, so experts 3..9 keep their first-pass count of 1
    assert m.admission == {**{i: 0 for i in range(3)}, **{i: 1 for i in range(3, 10)}}
    assert e.expert_of[:3] == [0, 1, 2]
    big = CacheModel(slots=0, margin_bytes=0)
    e2 = big.register("q", "t", 4096, 1, free_bytes=0)
    big.record(e2, None, [[i % 4096] for i in range(MISS_CAP + 10)])
    assert big.count == MISS_CAP + 10             # counter keeps counting
    big.step()
    assert big.last == (MISS_CAP, 0)              # the step reads at most MISS_CAP entries


@settings(max_examples=40, deadline=None)
@given(st.integers(0, 6), st.integers(1, 5), st.lists(st.lists(st.integers(0, 15), min_size=1, max_size=4), min_size=1,
                                                      max_size=30))
def test_model_invariants(slots, max_promo, trace):
    m = CacheModel(slots=slots, margin_bytes=0, max_promotions=max_promo)
    e = m.register("p", "t", 16, 1, free_bytes=1 << 40)
    g = m.register("g", "tg", 16, 1, free_bytes=1 << 40)
    for picks in trace:
        row = list(dict.fromkeys(picks))
        before = m.promotions
        m.record(e, g, [row])
        m.step()
        assert m.promotions - before <= max_promo
        for ent in (e, g):
            assert ent.n_slots == slots
            for s, ex in enumerate(ent.expert_of):       # slot_of / expert_of are inverse maps
                if ex >= 0:
                    assert ent.slot_of[ex] == s
            assert sum(1 for x in ent.slot_of if x >= 0) == sum(1 for x in ent.expert_of if x >= 0)
        assert all(v in (0, 1) for v in m.admission.values())
