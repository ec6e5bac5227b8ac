"""expert_cache_policy.py -- TEST INFRASTRUCTURE ONLY.

A plain-Python restatement of ExpertCache's residency policy
(/root/reference/core/expert_cache.{h,cpp}): pool signatures and sizing, the
LRU install, hits/misses/evictions, access counts, touch, ensure_resident and
the hot-profile file.  It moves no bytes: a "fetch" is recorded as the
(pool, slot, layer, expert, role) it would copy.  Only tests/ use it, as the
checker of libqwmoe's qwmoe_expert_cache_*; the product never imports it.

The reference class cannot be compiled here on its own (it needs the
reference's Model and ggml-backend objects), so this restatement is pinned by
tests/test_expert_cache.py against an independent LRU formulation (ordered
dictionaries), hand-worked traces and counting invariants.
"""
from __future__ import annotations

GATE, UP, DOWN = 0, 1, 2


class Pool:
    def __init__(self, role: int, type_: int, ne0: int, ne1: int, slab: int):
        self.role, self.type, self.ne0, self.ne1, self.slab = role, type_, ne0, ne1, slab
        self.n_layers = 0
        self.n_slots = 0
        self.key2slot: dict[int, int] = {}
        self.slot2key: list[int] = []
        self.clk: list[int] = []
        self.count: dict[int, int] = {}


class ExpertCachePolicy:
    """sigs: [role][layer] -> (type, ne0, ne1, slab bytes)."""

    def __init__(self, n_layer: int, n_expert: int, n_used: int, sigs, vram_budget: int):
        self.n_layer, self.n_expert, self.n_used = n_layer, n_expert, n_used
        self.pools: list[Pool] = []
        self.layer_pool = [[-1] * n_layer for _ in range(3)]
        # signature discovery: role outer, layer inner (expert_cache.cpp:128-152)
        for r in range(3):
            for il in range(n_layer):
                t, ne0, ne1, slab = sigs[r][il]
                idx = next((k for k, p in enumerate(self.pools)
                            if p.role == r and p.type == t and p.ne0 == ne0 and p.ne1 == ne1), -1)
                if idx < 0:
                    idx = len(self.pools)
                    self.pools.append(Pool(r, t, ne0, ne1, slab))
                self.pools[idx].n_layers += 1
                self.layer_pool[r][il] = idx
        # uniform residency fraction (expert_cache.cpp:155-186)
        total = sum(p.slab * p.n_layers * n_expert for p in self.pools)
        frac = vram_budget / total if total else 1.0
        frac = min(frac, 1.0)
        for p in self.pools:
            cap = p.n_layers * n_expert
            n = int(frac * cap)
            n = max(n, n_used)
            n = min(n, cap)
            p.n_slots = n
            p.slot2key = [-1] * n
            p.clk = [0] * n
        self.slot_of = [[0] * (n_layer * n_expert) for _ in range(3)]   # per role; 0 = absent
        self.clock = 0
        self.hits = self.misses = self.evictions = 0
        self.fetch_bytes = 0
        self.fetches: list[tuple] = []

    def pool(self, role: int, layer: int) -> Pool:
        return self.pools[self.layer_pool[role][layer]]

    def capacity(self, layer: int) -> int:               # expert_cache.cpp:288-293
        return min(self.pool(r, layer).n_slots for r in range(3))

    def min_slots(self) -> int:                          # expert_cache.cpp:282-286
        return min(p.n_slots for p in self.pools)

    def _install(self, role: int, layer: int, expert: int) -> int:   # expert_cache.cpp:374-391
        p = self.pool(role, layer)
        key = layer * self.n_expert + expert
        victim, best = 0, p.clk[0]
        for s in range(1, p.n_slots):
            if p.clk[s] < best:
                best, victim = p.clk[s], s
        old = p.slot2key[victim]
        if old >= 0:
            self.slot_of[role][old] = 0
            del p.key2slot[old]
            self.evictions += 1
        self.fetches.append((self.layer_pool[role][layer], victim, layer, expert, role))
        self.fetch_bytes += p.slab
        p.slot2key[victim] = key
        self.clock += 1
        p.clk[victim] = self.clock
        p.key2slot[key] = victim
        self.slot_of[role][key] = victim
        return victim

    def _slot_for(self, role: int, layer: int, expert: int) -> int:  # expert_cache.cpp:709-721
        p = self.pool(role, layer)
        key = layer * self.n_expert + expert
        p.count[key] = p.count.get(key, 0) + 1
        if key in p.key2slot:
            self.hits += 1
            self.clock += 1
            p.clk[p.key2slot[key]] = self.clock
            return p.key2slot[key]
        self.misses += 1
        return self._install(role, layer, expert)

    def ensure(self, layer: int, ids) -> tuple[list[int], list[int], list[int]]:   # expert_cache.cpp:790-832
        out = ([], [], [])
        for e in ids:
            for r in range(3):
                out[r].append(self._slot_for(r, layer, e))
        return out

    def ensure_resident(self, layer: int, expert: int) -> None:    # expert_cache.cpp:779-788
        key = layer * self.n_expert + expert
        for r in range(3):
            if key not in self.pool(r, layer).key2slot:
                self.misses += 1
                self._install(r, layer, expert)

    def touch(self, role: int, layer: int, expert: int) -> None:  # expert_cache.cpp:699-707
        p = self.pool(role, layer)
        key = layer * self.n_expert + expert
        if key not in p.key2slot:
            return
        p.count[key] = p.count.get(key, 0) + 1
        self.clock += 1
        p.clk[p.key2slot[key]] = self.clock
        self.hits += 1

    def verify(self, ids, touch: bool = True) -> int:
        """decode_cached_fast's residency check and accept (core/runtime.cpp:2922-2934,
        2959-2972): ids [n_layer][k]; entries absent in any role, touching all when none is."""
        missing = sum(1 for l, row in enumerate(ids) for e in row
                      if not all(self.resident(r, l, e) for r in range(3)))
        if missing == 0 and touch:
            for l, row in enumerate(ids):
                for e in row:
                    for r in range(3):
                        self.touch(r, l, e)
        return missing

    def resident(self, role: int, layer: int, expert: int) -> bool:
        return layer * self.n_expert + expert in self.pool(role, layer).key2slot

    def resmask(self, floor_res: int) -> tuple[list[list[float]], bool]:
        """decode_cached_fast's fill_resmask (core/runtime.cpp:2900-2919): 0 for an
        expert resident in all roles, -inf else; a layer with fewer than
        floor_res residents routes unmasked.  The floor is at least n_used (the
        reference's floor_res = max(n_used, ...), core/runtime.cpp:2896-2898).
        Returns (rows, complete)."""
        floor_res = max(floor_res, self.n_used)
        rows, complete = [], True
        for l in range(self.n_layer):
            res = [all(self.resident(r, l, e) for r in range(3)) for e in range(self.n_expert)]
            if sum(res) < floor_res:
                rows.append([0.0] * self.n_expert)
                complete = False
            else:
                rows.append([0.0 if x else float("-inf") for x in res])
        return rows, complete

    def refill(self, sel, want, budget: int, cursor: int) -> tuple[int, int]:
        """The background refill of a masked decode (core/runtime.cpp:2976-3008):
        touch the used experts, then fetch wanted-but-absent ones round robin
        from layer `cursor` within `budget`.  Returns (fetched, next cursor)."""
        if budget <= 0:
            return 0, cursor
        for l, row in enumerate(sel):
            for e in row:
                for r in range(3):
                    self.touch(r, l, e)
        fetched = 0
        for step in range(self.n_layer):
            if budget <= 0:
                break
            l = (cursor + step) % self.n_layer
            for e in want[l]:
                if budget <= 0:
                    break
                if all(self.resident(r, l, e) for r in range(3)):
                    continue
                self.ensure_resident(l, e)
                budget -= 1
                fetched += 1
        return fetched, (cursor + 1) % self.n_layer

    def slot_of_row(self, role: int, layer: int) -> list[int]:     # expert_cache.cpp:694-697
        return self.slot_of[role][layer * self.n_expert:(layer + 1) * self.n_expert]

    def profile_text(self) -> str:                                  # expert_cache.cpp:727-741
        lines = ["QWENEXPCACHE 1", f"{self.n_layer} {self.n_expert}"]
        for p in self.pools:
            for key in sorted(p.count):
                lines.append(f"{p.role} {key // self.n_expert} {key % self.n_expert} {p.count[key]}")
        return "\n".join(lines) + "\n"

    def load_prefetch(self, text: str) -> int:                      # expert_cache.cpp:743-777
        """Profile entries sorted by count, descending, equal counts in file order."""
        tok = text.split()
        if len(tok) < 4 or tok[0] != "QWENEXPCACHE" or tok[1] != "1":
            return 0
        if int(tok[2]) != self.n_layer or int(tok[3]) != self.n_expert:
            return 0
        ents = []
        rest = tok[4:]
        for i in range(0, len(rest) - 3, 4):
            r, l, e, c = (int(x) for x in rest[i:i + 4])
            if 0 <= r < 3 and 0 <= l < self.n_layer and 0 <= e < self.n_expert:
                ents.append((r, l, e, c))
        ents.sort(key=lambda x: -x[3])          # Python's sort is stable
        n = 0
        for r, l, e, _ in ents:
            p = self.pool(r, l)
            if len(p.key2slot) >= p.n_slots:
                continue
            if l * self.n_expert + e in p.key2slot:
                continue
            self._install(r, l, e)
            n += 1
        return n


def plan_slices(sel, n_used: int, n_expert: int, cap: int, max_slice: int = 1024):
    """plan_slices of the chunked prefill (core/runtime.cpp:2144-2170): cut the
    tokens' selections into slices naming at most cap distinct experts and at
    most max_slice tokens; returns ([(t0, len)], union in first-use order)."""
    if max_slice < 1:
        max_slice = 1024
    T = len(sel)
    slices, union, in_union = [], [], set()
    seen, distinct, t0 = set(), 0, 0
    for t in range(T):
        nnew = 0
        for e in sel[t]:
            if e not in in_union:
                in_union.add(e)
                union.append(e)
            if e not in seen:
                seen.add(e)
                nnew += 1
        if (distinct + nnew > cap or t - t0 >= max_slice) and t > t0:
            slices.append((t0, t - t0))
            seen, distinct = set(), 0
            nnew = 0
            for e in sel[t]:
                if e not in seen:
                    seen.add(e)
                    nnew += 1
            t0 = t
        distinct += nnew
    if T:
        slices.append((t0, T - t0))
    return slices, union
