"""Expert cache bookkeeping (CPU): the oracle's restatement of ExpertCache's
policy is pinned first (hand-worked traces, hand-computed pool sizes, an
independent LRU formulation, counting invariants); then libqwmoe's
qwmoe_expert_cache_* in a dry run (bookkeeping only, no device) must agree with
it call for call on random traces: slot ids, slot rows, residency, stats,
profile files and profile prefetch.
"""
from __future__ import annotations

import random
import sys
from collections import OrderedDict
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))

from expert_cache_policy import ExpertCachePolicy  # noqa: E402

Q8_0, Q4_K, Q6_K = 8, 12, 14
ROW = {Q8_0: lambda n: n // 32 * 34, Q4_K: lambda n: n // 256 * 144, Q6_K: lambda n: n // 256 * 210}


def sig(t, ne0, ne1):
    return (t, ne0, ne1, ROW[t](ne0) * ne1)


def uniform_sigs(n_layer, types=(Q4_K, Q4_K, Q6_K), H=256, F=256):
    shapes = ((H, F), (H, F), (F, H))
    return [[sig(types[r], *shapes[r]) for _ in range(n_layer)] for r in range(3)]


# ---- the oracle, pinned -------------------------------------------------------

def test_oracle_hand_worked_trace():
    """One layer, 4 experts, Q8_0 [32, 1] slabs (34 B): three pools (role is part
    of the signature), budget = half of 3*4*34 B -> 2 slots each."""
    sigs = [[sig(Q8_0, 32, 1)] for _ in range(3)]
    p = ExpertCachePolicy(1, 4, 1, sigs, 204)
    assert [q.n_slots for q in p.pools] == [2, 2, 2]
    got = [p.ensure(0, [e]) for e in (0, 1, 0, 2, 1)]
    # 0 -> slot 0, 1 -> slot 1, 0 hits slot 0, 2 evicts the LRU key 1 (slot 1),
    # 1 evicts the LRU key 0 (slot 0)
    assert [g[0][0] for g in got] == [0, 1, 0, 1, 0]
    assert all(g[0] == g[1] == g[2] for g in got)
    assert (p.hits, p.misses, p.evictions) == (3, 12, 6)
    assert p.fetch_bytes == 12 * 34
    # key 1 sits in slot 0, so its row entry equals the absent sentinel
    assert p.slot_of_row(0, 0) == [0, 0, 1, 0]
    assert [p.resident(0, 0, e) for e in range(4)] == [False, True, True, False]
    assert p.profile_text() == ("QWENEXPCACHE 1\n1 4\n" + "".join(
        f"{r} 0 0 2\n{r} 0 1 2\n{r} 0 2 1\n" for r in range(3)))
    # touch: a resident access (counts, stamps) ...
    p.touch(0, 0, 2)
    assert p.hits == 4 and p.pools[0].count[2] == 2
    # ... and a no-op when absent
    p.touch(0, 0, 3)
    assert p.hits == 4 and 3 not in p.pools[0].count
    # ensure_resident counts misses, not accesses: key 3 evicts key 1 from the
    # gate pool (key 2 was touched last) and key 2 from up and down (there key 1
    # was used after key 2)
    p.ensure_resident(0, 3)
    assert p.misses == 15 and p.evictions == 9
    assert p.slot_of_row(0, 0) == [0, 0, 1, 0] and p.resident(0, 0, 3) and not p.resident(0, 0, 1)
    assert p.resident(1, 0, 1) and not p.resident(1, 0, 2) and p.slot_of_row(1, 0)[3] == 1
    assert 3 not in p.pools[0].count


def test_oracle_pool_sizing_by_hand():
    """Two layers whose gate types differ: gate gets two pools, up and down one
    each (n_layers 2).  Slabs: Q4_K [256,256] = 36864 B, Q8_0 [256,256] = 69632 B,
    Q6_K [256,256] = 53760 B; E = 8."""
    sigs = [[sig(Q4_K, 256, 256), sig(Q8_0, 256, 256)],
            [sig(Q4_K, 256, 256)] * 2,
            [sig(Q6_K, 256, 256)] * 2]
    total = 8 * (36864 + 69632 + 2 * 36864 + 2 * 53760)     # 1 + 1 + 2 + 2 layers of 8 experts
    assert total == 2301952
    p = ExpertCachePolicy(2, 8, 2, sigs, total // 4)          # frac = 0.25 (575488 / 2301952)
    assert [(q.role, q.type, q.n_layers) for q in p.pools] == [(0, Q4_K, 1), (0, Q8_0, 1), (1, Q4_K, 2), (2, Q6_K, 2)]
    assert [q.n_slots for q in p.pools] == [2, 2, 4, 4]       # int(0.25 * 8) = 2, int(0.25 * 16) = 4
    assert p.layer_pool == [[0, 1], [2, 2], [3, 3]]
    assert p.capacity(0) == 2 and p.min_slots() == 2
    p = ExpertCachePolicy(2, 8, 3, sigs, total // 4)          # the n_used floor
    assert [q.n_slots for q in p.pools] == [3, 3, 4, 4]
    p = ExpertCachePolicy(2, 8, 3, sigs, 10 * total)          # capped at every expert
    assert [q.n_slots for q in p.pools] == [8, 8, 16, 16]
    p = ExpertCachePolicy(2, 8, 3, sigs, 0)
    assert [q.n_slots for q in p.pools] == [3, 3, 3, 3]


class OrderedLru:
    """The same policy written another way: per pool, resident keys in recency
    order (OrderedDict) and the free slots; a miss takes the lowest free slot,
    else evicts the least recently used key."""

    def __init__(self, ref: ExpertCachePolicy):
        self.E = ref.n_expert
        self.layer_pool = ref.layer_pool
        self.pools = [{"lru": OrderedDict(), "free": list(range(q.n_slots)), "count": {}} for q in ref.pools]
        self.hits = self.misses = self.evictions = 0

    def _install(self, q, key):
        if q["free"]:
            slot = min(q["free"])
            q["free"].remove(slot)
        else:
            _, slot = q["lru"].popitem(last=False)
            self.evictions += 1
        q["lru"][key] = slot
        return slot

    def access(self, r, l, e, count=True):
        q = self.pools[self.layer_pool[r][l]]
        key = l * self.E + e
        if count:
            q["count"][key] = q["count"].get(key, 0) + 1
        if key in q["lru"]:
            q["lru"].move_to_end(key)
            self.hits += 1
            return q["lru"][key]
        self.misses += 1
        return self._install(q, key)

    def ensure(self, l, ids):
        out = ([], [], [])
        for e in ids:
            for r in range(3):
                out[r].append(self.access(r, l, e))
        return out

    def touch(self, r, l, e):
        q = self.pools[self.layer_pool[r][l]]
        if l * self.E + e in q["lru"]:
            self.access(r, l, e)

    def ensure_resident(self, l, e):
        for r in range(3):
            q = self.pools[self.layer_pool[r][l]]
            key = l * self.E + e
            if key not in q["lru"]:
                self.misses += 1
                self._install(q, key)

    def row(self, r, l):
        q = self.pools[self.layer_pool[r][l]]
        out = [0] * self.E
        for key, slot in q["lru"].items():
            if key // self.E == l:
                out[key % self.E] = slot
        return out


def random_setup(rng: random.Random):
    n_layer = rng.randint(1, 5)
    E = rng.choice([8, 16, 32])
    n_used = rng.randint(1, min(4, E))
    choices = [(Q4_K, Q4_K, Q6_K), (Q8_0, Q8_0, Q4_K), (Q4_K, Q4_K, Q4_K)]
    per_layer = [rng.choice(choices) for _ in range(n_layer)]
    sigs = [[sig(per_layer[l][r], 256, 256) for l in range(n_layer)] for r in range(3)]
    total = sum(s[3] for r in range(3) for s in sigs[r]) * E
    budget = int(total * rng.choice([0.0, 0.1, 0.3, 0.5, 0.9, 1.5]))
    return n_layer, E, n_used, sigs, budget


def zipf_ids(rng, E, k, s=1.1):
    w = [1.0 / (i + 1) ** s for i in range(E)]
    perm = list(range(E))
    rng.shuffle(perm)
    out = []
    while len(out) < k:
        e = perm[rng.choices(range(E), weights=w)[0]]
        if e not in out:
            out.append(e)
    return out


def random_ops(rng, p: ExpertCachePolicy, n_ops: int):
    ops = []
    for _ in range(n_ops):
        l = rng.randrange(p.n_layer)
        u = rng.random()
        if u < 0.7:
            k = rng.randint(1, min(p.capacity(l), p.n_expert))
            ids = zipf_ids(rng, p.n_expert, k)
            if rng.random() < 0.2:
                ids = ids + [rng.choice(ids)]                     # a repeat within one call hits
            ops.append(("ensure", l, ids))
        elif u < 0.8:
            ops.append(("touch", rng.randrange(3), l, rng.randrange(p.n_expert)))
        elif u < 0.9:
            ops.append(("ensure_resident", l, rng.randrange(p.n_expert)))
        else:
            k = min(p.n_expert, 4)
            ids = [zipf_ids(rng, p.n_expert, k) for _ in range(rng.randint(1, p.n_layer))]
            ops.append(("verify", ids))
    return ops


def apply_both(c, p, op):
    if op[0] == "ensure":
        assert c.ensure(op[1], op[2]) == p.ensure(op[1], op[2])
    elif op[0] == "touch":
        c.touch(*op[1:])
        p.touch(*op[1:])
    elif op[0] == "verify":
        import numpy as np
        assert c.verify(np.array(op[1], np.int32)) == p.verify(op[1])
    else:
        c.ensure_resident(*op[1:])
        p.ensure_resident(*op[1:])


@pytest.mark.parametrize("seed", range(40))
def test_oracle_matches_ordered_lru(seed):
    rng = random.Random(seed)
    n_layer, E, n_used, sigs, budget = random_setup(rng)
    p = ExpertCachePolicy(n_layer, E, n_used, sigs, budget)
    q = OrderedLru(p)
    accesses = 0
    for op in random_ops(rng, p, 300):
        if op[0] == "ensure":
            assert p.ensure(op[1], op[2]) == q.ensure(op[1], op[2])
            accesses += 3 * len(op[2])
        elif op[0] == "touch":
            p.touch(*op[1:])
            q.touch(*op[1:])
        elif op[0] == "verify":
            miss = sum(1 for l, row in enumerate(op[1]) for e in row
                       if any(l * q.E + e not in q.pools[q.layer_pool[r][l]]["lru"] for r in range(3)))
            assert p.verify(op[1]) == miss
            if miss == 0:
                for l, row in enumerate(op[1]):
                    for e in row:
                        for r in range(3):
                            q.touch(r, l, e)
        else:
            p.ensure_resident(*op[1:])
            q.ensure_resident(*op[1:])
        for r in range(3):
            for l in range(n_layer):
                assert p.slot_of_row(r, l) == q.row(r, l)
    assert (p.hits, p.misses, p.evictions) == (q.hits, q.misses, q.evictions)
    # counting invariants
    assert p.fetch_bytes == sum(p.pools[f[0]].slab for f in p.fetches) and len(p.fetches) == p.misses
    filled = sum(sum(1 for k in pool.slot2key if k >= 0) for pool in p.pools)
    assert p.evictions == p.misses - filled
    for pool, qq in zip(p.pools, q.pools):
        assert pool.count == qq["count"]
        assert len(pool.key2slot) <= pool.n_slots


# ---- the library against the oracle ------------------------------------------------

def lib_or_skip():
    from questwend_amd import LIB_PATH
    if not LIB_PATH.exists():
        pytest.skip("libqwmoe.so not built")
    from questwend_amd import ops
    return ops


def make_lib(ops, n_layer, E, n_used, sigs, budget):
    srcs = [[{"type": sigs[r][l][0], "ne0": sigs[r][l][1], "ne1": sigs[r][l][2], "host": 1}
             for l in range(n_layer)] for r in range(3)]
    return ops.ExpertCache(n_layer, E, srcs, budget, n_used, dry_run=True)


def assert_same(c, p: ExpertCachePolicy):
    st = c.stats()
    assert (st["hits"], st["misses"], st["evictions"], st["fetch_bytes"]) == (p.hits, p.misses, p.evictions,
                                                                               p.fetch_bytes)
    for r in range(3):
        for l in range(p.n_layer):
            assert c.slot_of_row(r, l) == p.slot_of_row(r, l)
            for e in range(p.n_expert):
                assert c.resident(r, l, e) == p.resident(r, l, e)


@pytest.mark.parametrize("seed", range(25))
def test_library_matches_oracle(seed, tmp_path):
    ops = lib_or_skip()
    rng = random.Random(1000 + seed)
    n_layer, E, n_used, sigs, budget = random_setup(rng)
    p = ExpertCachePolicy(n_layer, E, n_used, sigs, budget)
    c = make_lib(ops, n_layer, E, n_used, sigs, budget)
    pools = c.pools()
    assert [(x["role"], x["type"], x["n_slots"], x["slab"]) for x in pools] == \
        [(q.role, q.type, q.n_slots, q.slab) for q in p.pools]
    assert all(x["base"] is None or x["base"] == 0 for x in pools)           # a dry run has no device pools
    assert c.min_slots() == p.min_slots()
    for l in range(n_layer):
        assert c.capacity(l) == p.capacity(l)
        for r in range(3):
            assert c.pool_of(r, l) == p.layer_pool[r][l]
    for op in random_ops(rng, p, 250):
        apply_both(c, p, op)
    assert_same(c, p)
    # profile file: byte for byte
    prof = tmp_path / "hot.txt"
    c.save_profile(prof)
    assert prof.read_text() == p.profile_text()
    # prefetch into fresh caches, then both keep going
    c2 = make_lib(ops, n_layer, E, n_used, sigs, budget)
    p2 = ExpertCachePolicy(n_layer, E, n_used, sigs, budget)
    assert c2.load_prefetch(prof) == p2.load_prefetch(prof.read_text())
    assert_same(c2, p2)
    for op in random_ops(rng, p2, 100):
        apply_both(c2, p2, op)
    assert_same(c2, p2)


def test_prefetch_order_and_fill(tmp_path):
    """Hottest keys first, equal counts in file order, each pool up to its size,
    entries out of range ignored; a missing or mismatched profile prefetches
    nothing."""
    ops = lib_or_skip()
    sigs = uniform_sigs(2)
    total = 2 * 8 * sum(sigs[r][0][3] for r in range(3))
    budget = total * 3 // 8                   # 3 of 8 experts per layer -> 6 slots per pool
    c = make_lib(ops, 2, 8, 2, sigs, budget)
    p = ExpertCachePolicy(2, 8, 2, sigs, budget)
    assert [x["n_slots"] for x in c.pools()] == [6, 6, 6]
    text = "QWENEXPCACHE 1\n2 8\n" + "".join(
        f"{r} {l} {e} {cnt}\n" for r, l, e, cnt in
        [(0, 0, 1, 5), (0, 0, 2, 9), (0, 1, 7, 5), (0, 0, 3, 5), (0, 1, 0, 1), (0, 0, 4, 5), (0, 0, 5, 5),
         (0, 1, 6, 5), (1, 0, 0, 3), (2, 9, 0, 100), (3, 0, 0, 100), (0, 0, 8, 100), (2, 1, 1, 2)])
    f = tmp_path / "p.txt"
    f.write_text(text)
    n = c.load_prefetch(f)
    assert n == p.load_prefetch(text) == 6 + 1 + 1
    assert_same(c, p)
    # gate: 2 (count 9), then the count-5 keys in file order: 0:1, 1:7, 0:3, 0:4, 0:5 -> pool full (6)
    assert p.slot_of_row(0, 0)[2] == 0 and p.slot_of_row(0, 0)[1] == 1 and p.slot_of_row(0, 1)[7] == 2
    assert not p.resident(0, 1, 6) and not p.resident(0, 1, 0)
    st = c.stats()
    assert st["misses"] == 0 and st["evictions"] == 0
    assert st["fetch_bytes"] == 7 * sigs[0][0][3] + sigs[2][0][3]     # 6 gate + 1 up slabs, 1 down slab
    for bad in ["", "QWENEXPCACHE 2\n2 8\n0 0 0 1\n", "QWENEXPCACHE 1\n3 8\n0 0 0 1\n", "NOPE 1\n2 8\n"]:
        f.write_text(bad)
        c3 = make_lib(ops, 2, 8, 2, sigs, budget)
        assert c3.load_prefetch(f) == 0
    c3 = make_lib(ops, 2, 8, 2, sigs, budget)
    assert c3.load_prefetch(tmp_path / "missing.txt") == 0


def test_ensure_rejects_over_capacity_and_bad_ids():
    ops = lib_or_skip()
    from questwend_amd import QwmoeError
    sigs = uniform_sigs(1)
    c = make_lib(ops, 1, 16, 2, sigs, 0)           # 2 slots per pool
    assert c.capacity(0) == 2
    c.ensure(0, [3, 3, 5])                          # two distinct experts fit
    before = c.stats()
    for ids in ([1, 2, 3], [16], [-1]):
        with pytest.raises(QwmoeError):
            c.ensure(0, ids)
    assert c.stats() == before                      # nothing changed
    with pytest.raises(QwmoeError):
        c.ensure_resident(1, 0)
    with pytest.raises(QwmoeError):
        c.touch(3, 0, 0)
    with pytest.raises(ValueError):
        c.slot_of_row(0, 1)
    with pytest.raises(QwmoeError):
        c.layer(0)                                  # a dry run has no device pools


def test_create_rejects_bad_sources():
    ops = lib_or_skip()
    from questwend_amd import QwmoeError
    sigs = uniform_sigs(1)
    good = [[{"type": sigs[r][0][0], "ne0": sigs[r][0][1], "ne1": sigs[r][0][2], "host": 1}] for r in range(3)]
    ops.ExpertCache(1, 8, good, 0, 2, dry_run=True)
    for mutate in (lambda s: s[0][0].update(type=0), lambda s: s[1][0].update(ne0=100),
                   lambda s: s[2][0].update(host=None), lambda s: s[0][0].update(ne1=0)):
        bad = [[dict(x) for x in row] for row in good]
        mutate(bad)
        with pytest.raises(QwmoeError):
            ops.ExpertCache(1, 8, bad, 0, 2, dry_run=True)
    with pytest.raises(QwmoeError):
        ops.ExpertCache(1, 8, good, 0, 9, dry_run=True)          # n_used > n_expert


def test_gguf_pools_dry(tmp_path):
    """Pools of a GGUF model as ExpertCache builds them: the single-file fixture
    has layer 0 (Q4_K, Q4_K, Q6_K) and layer 1 (Q8_0, Q8_0, Q4_K), so six
    pools of one layer each; the shard set's layer spans both files."""
    ops = lib_or_skip()
    sys.path.insert(0, str(ROOT / "tests"))
    import gguf_fixtures as FX
    from oracle_lib import Oracle
    FX.write_all(tmp_path, Oracle())
    with ops.Gguf(tmp_path / "moe_tiny.gguf") as g:
        for tier in (0, 1):
            c = ops.ExpertCache.from_gguf(g, tier, 0, dry_run=True)
            pools = c.pools()
            assert [(x["role"], x["type"]) for x in pools] == [(0, Q4_K), (0, Q8_0), (1, Q4_K), (1, Q8_0),
                                                               (2, Q6_K), (2, Q4_K)]
            assert all(x["n_slots"] == FX.K_USED for x in pools)
            assert c.capacity(1) == FX.K_USED
            c.close()
        c = ops.ExpertCache.from_gguf(g, 1, 10 ** 12, n_used=1, dry_run=True)
        assert [x["n_slots"] for x in c.pools()] == [FX.E] * 6
    with ops.Gguf(tmp_path / "moe_split-00001-of-00002.gguf") as g:
        c = ops.ExpertCache.from_gguf(g, 1, 0, dry_run=True)
        assert [(x["role"], x["type"], x["ne0"], x["ne1"]) for x in c.pools()] == \
            [(0, Q4_K, FX.H, FX.F_EXP), (1, Q4_K, FX.H, FX.F_EXP), (2, Q4_K, FX.F_EXP, FX.H)]


def test_run_layer_needs_device_pools():
    ops = lib_or_skip()
    from questwend_amd import Layer, QwmoeError
    sigs = uniform_sigs(1)
    c = make_lib(ops, 1, 16, 2, sigs, 0)
    import ctypes as C
    L = Layer()
    L.n_embd, L.n_expert, L.n_expert_used, L.n_ff = 256, 16, 2, 256
    rc = ops.lib().qwmoe_expert_cache_run_layer(c.h, 0, C.byref(L), 1, 1, 1, -1.0, None, None, None)
    assert rc != 0
    with pytest.raises(QwmoeError):
        ops.check(rc, "run_layer")


# ---- resident-only decode: the mask and the background refill ----------------------

def test_oracle_resmask_and_refill_by_hand():
    """Pins the policy's fill_resmask / refill (core/runtime.cpp:2900-2919,
    2976-3008) on a worked case: 2 layers x 4 experts, one pool per role with 4
    slots shared by both layers (LRU across them)."""
    sigs = uniform_sigs(2)
    p = ExpertCachePolicy(2, 4, 2, sigs, sum(sigs[r][0][3] for r in range(3)) * 2 * 4 // 2)   # half of everything
    assert [q.n_slots for q in p.pools] == [4, 4, 4]
    p.ensure(0, [1, 3])
    p.ensure(1, [2])
    ninf = float("-inf")
    rows, complete = p.resmask(floor_res=2)                   # layer 1 has one resident: left unmasked
    assert rows[0] == [ninf, 0.0, ninf, 0.0] and rows[1] == [0.0] * 4 and not complete
    assert p.resmask(floor_res=1) == (rows, complete)         # the floor is at least n_used (2)
    q = ExpertCachePolicy(2, 4, 2, sigs, sum(sigs[r][0][3] for r in range(3)) * 2 * 4 // 2)
    q.ensure(0, [1, 3])
    q.ensure(1, [2, 3])
    assert q.resmask(floor_res=0) == ([[ninf, 0.0, ninf, 0.0], [ninf, ninf, 0.0, 0.0]], True)
    # refill from layer 1 (cursor 1), budget 2: the used experts are touched in
    # order (0,1), (0,3), (1,2); layer 1 wants 0 (a free slot) then 3 (evicts the
    # least recently used, (0,1))
    misses, evictions = p.misses, p.evictions
    fetched, cur = p.refill(sel=[[1, 3], [2, 2]], want=[[0, 1], [0, 3]], budget=2, cursor=1)
    assert (fetched, cur) == (2, 0)
    assert (p.misses, p.evictions) == (misses + 6, evictions + 3)     # 2 experts x 3 roles; one eviction per pool
    assert all(p.resident(r, 1, e) for r in range(3) for e in (0, 2, 3))
    assert all(p.resident(r, 0, 3) for r in range(3)) and not any(p.resident(r, 0, 1) for r in range(3))
    assert p.refill([[3, 3], [0, 3]], [[0, 1], [0, 3]], budget=0, cursor=0) == (0, 0)


@pytest.mark.parametrize("seed", range(12))
def test_library_resident_helpers_match_oracle(seed):
    """qwmoe_expert_cache_resmask / _refill (dry run) against the policy, call for
    call, interleaved with the other operations; state compared after each."""
    import numpy as np
    ops = lib_or_skip()
    rng = random.Random(5000 + seed)
    n_layer, E, n_used, sigs, budget = random_setup(rng)
    p = ExpertCachePolicy(n_layer, E, n_used, sigs, budget)
    c = make_lib(ops, n_layer, E, n_used, sigs, budget)
    cursor = 0
    for _ in range(12):
        for op in random_ops(rng, p, 20):
            apply_both(c, p, op)
        floor = rng.randint(0, E)
        m, complete = c.resmask(floor)
        rows, comp2 = p.resmask(floor)
        assert complete == comp2
        assert np.array_equal(m, np.array(rows, np.float32))
        k = min(n_used, E)
        sel = [zipf_ids(rng, E, k) for _ in range(n_layer)]
        want = [zipf_ids(rng, E, k) for _ in range(n_layer)]
        b = rng.randint(0, 6)
        got = c.refill(np.array(sel, np.int32), np.array(want, np.int32), b, cursor)
        exp = p.refill(sel, want, b, cursor)
        assert got == exp
        cursor = got[1]
        assert_same(c, p)


# ---- batch slicing against pool capacity -----------------------------------------

def test_oracle_plan_slices_by_hand():
    """plan_slices (core/runtime.cpp:2144-2170) on a worked case: n_used 2, cap 3.
    t0 {0,1} -> 2 distinct; t1 {1,2} -> 3; t2 {3,0} would make 5 > 3: slice
    (0, 2) closes, t2 opens with {3,0}; t3 {0,3} -> still 2; t4 {4,5} -> 4 > 3:
    (2, 2) closes; t4 alone -> (4, 1).  max_slice 2 caps lengths instead."""
    from expert_cache_policy import plan_slices
    sel = [[0, 1], [1, 2], [3, 0], [0, 3], [4, 5]]
    assert plan_slices(sel, 2, 6, 3) == ([(0, 2), (2, 2), (4, 1)], [0, 1, 2, 3, 4, 5])
    assert plan_slices(sel, 2, 6, 10, max_slice=2) == ([(0, 2), (2, 2), (4, 1)], [0, 1, 2, 3, 4, 5])
    assert plan_slices(sel, 2, 6, 10) == ([(0, 5)], [0, 1, 2, 3, 4, 5])
    assert plan_slices([], 2, 6, 3) == ([], [])


@pytest.mark.parametrize("seed", range(20))
def test_library_plan_slices_matches_oracle(seed):
    import numpy as np
    from expert_cache_policy import plan_slices
    ops = lib_or_skip()
    rng = random.Random(7000 + seed)
    E = rng.choice([8, 16, 32, 128])
    n_used = rng.randint(1, min(8, E))
    T = rng.randint(0, 300)
    cap = rng.randint(n_used, E + 4)
    max_slice = rng.choice([0, 1, 3, 17, 1024])
    sel = [zipf_ids(rng, E, n_used) for _ in range(T)]
    got = ops.plan_slices(np.array(sel, np.int32).reshape(T, n_used), E, cap, max_slice)
    assert got == plan_slices(sel, n_used, E, cap, max_slice)
    # every slice fits the cap and the max length, and they tile the tokens
    sl, _ = got
    assert sum(n for _, n in sl) == T and all(n <= (max_slice if max_slice >= 1 else 1024) for _, n in sl)
    assert all(len({e for t in range(t0, t0 + n) for e in sel[t]}) <= cap for t0, n in sl)
