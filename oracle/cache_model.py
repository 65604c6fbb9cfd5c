"""Model of the hot-expert cache state machine (TEST INFRASTRUCTURE ONLY).

Restates, independently of the product's C++, the reference's host logic and
the recorder contract of its kernel:
  * registration and pool sizing      kernels/moe-cache.cu:525-622
  * seed file parsing                 kernels/moe-cache.cu:483-523
  * pick recording (stamps, counters,
    miss log packing cid<<12|expert)  kernels/moe-cache.cu:159-204
  * slot acquisition / LRU eviction   kernels/moe-cache.cu:628-667
  * the between-graph step            kernels/moe-cache.cu:669-775
The one deliberate difference from the reference is the miss-log ORDER: the
reference appends with atomicAdd across thread blocks (racy); the model, like
the product, writes entries in pick order (token-major, slot, up before gate),
one of the orders the reference can produce.  tests/test_cache_model.py pins
the model with hand-derived scenarios and invariants.
"""
from __future__ import annotations

from dataclasses import dataclass, field

MISS_CAP = 8190
GIB = 1 << 30


def parse_seed_text(text: str) -> dict:
    """'name id,id,...' per line; a line without a space is skipped; parsing of a line
    stops at the first token that is not an integer (strtol semantics); a later line for
    the same name replaces the earlier one."""
    seed = {}
    for raw in text.splitlines(keepends=True):
        if " " not in raw:
            continue
        name, rest = raw.split(" ", 1)
        ids = []
        p = rest
        while p:
            i = 0
            # strtol: optional leading whitespace, sign, digits
            while i < len(p) and p[i] in " \t\n\r\f\v":
                i += 1
            j = i
            if j < len(p) and p[j] in "+-":
                j += 1
            k = j
            while k < len(p) and p[k].isdigit():
                k += 1
            if k == j:
                break
            ids.append(int(p[i:k]))
            p = p[k + 1:] if k < len(p) and p[k] == "," else p[k:]
        seed[name] = ids
    return seed


def parse_seed_file(path) -> dict:
    with open(path, "r") as f:
        return parse_seed_text(f.read())


@dataclass
class Entry:
    id: int
    name: str
    n_experts: int
    expert_bytes: int
    n_slots: int
    slot_of: list = field(default_factory=list)      # expert -> slot / -1
    expert_of: list = field(default_factory=list)    # slot -> expert / -1
    stamps: list = field(default_factory=list)       # device stamps
    h_stamps: list = field(default_factory=list)     # host mirror
    stamps_clock: int = 0
    tbl_dirty: bool = False

    def table(self):
        """Decoded pointer table: slot index for LSB=0 entries, -1 for host entries."""
        return list(self.slot_of)


class CacheModel:
    def __init__(self, slots=-1, budget_bytes=0, margin_bytes=2 * GIB, max_promotions=48, seed=None):
        self.cfg_slots = slots
        self.budget = budget_bytes
        self.margin = margin_bytes
        self.max_promotions = max_promotions
        self.seed = seed or {}
        self.entries: list[Entry] = []
        self.by_key = {}
        self.used = 0
        self.clock = 0
        self.d_clock = 0
        self.count = 0           # stats[0]
        self.hits = 0            # stats[1]
        self.log = [0] * MISS_CAP
        self.admission = {}
        self.promotions = 0
        self.evictions = 0
        self.steps = 0

    # -- registration -------------------------------------------------------
    def register(self, key, name, n_experts, expert_bytes, free_bytes):
        if key in self.by_key:
            return self.by_key[key]
        slots = n_experts if self.cfg_slots < 0 else self.cfg_slots
        if self.budget > 0:
            free_budget = max(self.budget - self.used, 0)
            if slots * expert_bytes > free_budget:
                slots = free_budget // expert_bytes
        usable = free_bytes - self.margin if free_bytes > self.margin else 0
        if slots * expert_bytes > usable:
            slots = usable // expert_bytes
        slots = min(slots, n_experts)
        e = Entry(id=len(self.entries), name=name, n_experts=n_experts, expert_bytes=expert_bytes, n_slots=slots,
                  slot_of=[-1] * n_experts, expert_of=[-1] * slots, stamps=[0] * n_experts,
                  h_stamps=[0] * n_experts)
        if slots > 0:
            self.used += slots * expert_bytes
        self.entries.append(e)
        self.by_key[key] = e
        seeded = 0
        for ex in self.seed.get(name, []):
            if seeded >= e.n_slots:
                break
            if ex < 0 or ex >= n_experts or e.slot_of[ex] >= 0:
                continue
            e.slot_of[ex] = seeded
            e.expert_of[seeded] = ex
            seeded += 1
        return e

    # -- the kernel's recorder ---------------------------------------------
    def record(self, up: Entry, gate: Entry | None, ids):
        """ids: [n_tok][n_used] expert ids of one GEMV launch."""
        for row in ids:
            for ex in row:
                if ex < 0 or ex >= up.n_experts:
                    continue
                up.stamps[ex] = self.d_clock
                self._one(up, ex)
                if gate is not None:
                    gate.stamps[ex] = self.d_clock
                    self._one(gate, ex)

    def _one(self, e: Entry, ex: int):
        if e.slot_of[ex] < 0:            # LSB=1: host entry -> miss
            s = self.count
            self.count += 1
            if s < MISS_CAP:
                self.log[s] = (e.id << 12) | ex
        else:
            self.hits += 1

    # -- LRU step -----------------------------------------------------------
    def _acquire(self, e: Entry) -> int:
        if e.n_slots == 0:
            return -1
        for s in range(e.n_slots):
            if e.expert_of[s] < 0:
                return s
        if e.stamps_clock != self.clock:
            e.h_stamps = list(e.stamps)
            e.stamps_clock = self.clock
        victim, best = -1, 0xFFFFFFFF
        for s in range(e.n_slots):
            ex = e.expert_of[s]
            st = e.h_stamps[ex] if ex >= 0 else 0
            if st < best:
                best, victim = st, s
        if victim < 0:
            return -1
        v = e.expert_of[victim]
        if v >= 0:
            e.slot_of[v] = -1
            e.tbl_dirty = True
            self.evictions += 1
        e.expert_of[victim] = -1
        return victim

    def step(self):
        n = min(self.count, MISS_CAP)
        step_hits = self.hits
        self.clock += 1
        self.d_clock = self.clock
        self.count = 0
        self.hits = 0
        self.steps += 1
        self.last = (n, step_hits)
        if n == 0:
            return
        promoted = 0
        i = 0
        while i < n and promoted < self.max_promotions:
            packed = self.log[i]
            i += 1
            cid, ex = packed >> 12, packed & 0xFFF
            c = self.admission.get(packed, 0) + 1
            self.admission[packed] = c
            if c < 2:
                continue
            self.admission[packed] = 0
            if cid < 0 or cid >= len(self.entries):
                continue
            e = self.entries[cid]
            if ex < 0 or ex >= e.n_experts or e.slot_of[ex] >= 0:
                continue
            slot = self._acquire(e)
            if slot < 0:
                continue
            e.slot_of[ex] = slot
            e.expert_of[slot] = ex
            e.tbl_dirty = True
            promoted += 1
            self.promotions += 1
        for e in self.entries:
            e.tbl_dirty = False
        if len(self.admission) > 8192:
            self.admission = {k: v for k, v in self.admission.items() if v != 0}
