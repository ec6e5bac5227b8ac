"""GPU parity of the expert cache (qwmoe_expert_cache_*).

* Pool contents: after every call, each occupied slot of each pool holds
  exactly the bytes of its (layer, expert) slab in the source tier -- pinned
  host memory, a GGUF file read by the file tier, or the GGUF host tier's
  pinned copy -- and the device slot rows equal the host rows, which equal the
  oracle's (oracle/expert_cache_policy.py).
* Results: one MoE FFN layer computed through the cache's pools and rows
  (qwmoe_ffn_layer) is bit-identical to the same layer on the all-resident
  tensors; a decode stack over the cache speculates on the resident set,
  verifies the ids it used, falls back layer by layer with ensure() on a miss
  (core/runtime.cpp:2921-2933, 2458-2662), and every token's output is
  bit-identical to the all-resident stack's.
"""
from __future__ import annotations

import ctypes as C
import random
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "oracle"))
import questwend_amd as qa  # noqa: E402
from questwend_amd import ops  # noqa: E402
from expert_cache_policy import ExpertCachePolicy  # noqa: E402
from oracle_lib import Q4_K, Q6_K, Q8_0, Oracle, row_size  # noqa: E402

DEV = "cuda:0"


def note(msg: str) -> None:
    print(f"[gpu-expert-cache] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    prev = ops.set_mfma_form(ops.MFMA_EXACT)   # bit-exact tests: heavy bins on the matrix cores replay ggml's float steps
    yield
    torch.cuda.synchronize()
    ops.set_mfma_form(prev)


_hip = None


def d2h(ptr: int, n: int) -> bytes:
    """n bytes at device address ptr (hipMemcpy, device to host)."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.restype = C.c_int
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    buf = (C.c_uint8 * n)()
    assert _hip.hipMemcpy(buf, C.c_void_p(ptr), n, 2) == 0
    return bytes(buf)


def check_pools(cache, p: ExpertCachePolicy, slab_bytes):
    """slab_bytes(role, layer, expert) -> the source bytes."""
    cache.sync()
    pools = cache.pools()
    for pi, (info, pol) in enumerate(zip(pools, p.pools)):
        assert info["n_slots"] == pol.n_slots and info["slab"] == pol.slab
        raw = d2h(info["base"], info["n_slots"] * info["slab"])
        for s, key in enumerate(pol.slot2key):
            if key < 0:
                continue
            l, e = divmod(key, p.n_expert)
            got = raw[s * info["slab"]:(s + 1) * info["slab"]]
            assert got == slab_bytes(pol.role, l, e), f"pool {pi} slot {s}: layer {l} expert {e}"
    for r in range(3):
        for l in range(p.n_layer):
            row = cache.slot_of_row(r, l)
            assert row == p.slot_of_row(r, l), f"host row {r}/{l}"
            dev = np.frombuffer(d2h(cache.device_row(r, l), 4 * p.n_expert), np.int32)
            assert dev.tolist() == row, f"device row {r}/{l}"
    st = cache.stats()
    assert (st["hits"], st["misses"], st["evictions"], st["fetch_bytes"]) == (p.hits, p.misses, p.evictions,
                                                                               p.fetch_bytes)


def random_trace(rng, p, n):
    ops_ = []
    for _ in range(n):
        l = rng.randrange(p.n_layer)
        u = rng.random()
        if u < 0.75:
            k = rng.randint(1, min(p.capacity(l), p.n_expert))
            ops_.append(("ensure", l, rng.sample(range(p.n_expert), k)))
        elif u < 0.85:
            ops_.append(("touch", rng.randrange(3), l, rng.randrange(p.n_expert)))
        elif u < 0.95:
            ops_.append(("ensure_resident", l, rng.randrange(p.n_expert)))
        else:
            ops_.append(("verify", [rng.sample(range(p.n_expert), min(2, p.n_expert)) for _ in range(p.n_layer)]))
    return ops_


def apply(cache, p, op):
    if op[0] == "ensure":
        assert cache.ensure(op[1], op[2]) == p.ensure(op[1], op[2])
    elif op[0] == "touch":
        cache.touch(*op[1:])
        p.touch(*op[1:])
    elif op[0] == "verify":
        assert cache.verify(np.array(op[1], np.int32)) == p.verify(op[1])
    else:
        cache.ensure_resident(*op[1:])
        p.ensure_resident(*op[1:])


@pytest.mark.parametrize("source", ["pinned", "pinned-copy-engine", "pageable"])
def test_host_tier_pool_bytes(tmp_path, source):
    """Three layers (two signatures), 16 experts, random slabs, 30% resident.
    Pinned sources send scattered misses through the slab gather kernel (or,
    with QWMOE_CACHE_COPY_ENGINE, the copy engine); pageable ones always use
    the copy engine."""
    note(f"host tier ({source}): 3 layers, 16 experts, 30% resident, 120 calls + profile prefetch")
    H, F, E, n_used = 256, 512, 16, 2
    types = [(Q4_K, Q4_K, Q6_K), (Q8_0, Q8_0, Q4_K), (Q4_K, Q4_K, Q6_K)]
    shapes = ((H, F), (H, F), (F, H))
    g = torch.Generator().manual_seed(7)
    src, sigs = [[None] * 3 for _ in range(3)], [[None] * 3 for _ in range(3)]
    for r in range(3):
        for l in range(3):
            t, (ne0, ne1) = types[l][r], shapes[r]
            slab = row_size(t, ne0) * ne1
            host = torch.randint(0, 256, (E * slab,), dtype=torch.uint8, generator=g)
            if source != "pageable":
                host = host.pin_memory()
            src[r][l] = host
            sigs[r][l] = (t, ne0, ne1, slab)
    total = sum(sigs[r][l][3] for r in range(3) for l in range(3)) * E
    budget = int(total * 0.3)
    srcs = [[{"type": sigs[r][l][0], "ne0": sigs[r][l][1], "ne1": sigs[r][l][2], "host": src[r][l].data_ptr()}
             for l in range(3)] for r in range(3)]
    ce = source == "pinned-copy-engine"
    cache = ops.ExpertCache(3, E, srcs, budget, n_used, copy_engine=ce)
    p = ExpertCachePolicy(3, E, n_used, sigs, budget)

    def slab_bytes(r, l, e):
        n = sigs[r][l][3]
        return src[r][l][e * n:(e + 1) * n].numpy().tobytes()

    check_pools(cache, p, slab_bytes)                      # empty pools, rows all 0
    # consecutive experts into consecutive empty slots: merged into one copy per pool
    apply(cache, p, ("ensure", 0, [0, 1, 2, 3]))
    apply(cache, p, ("ensure", 2, [5, 6, 9]))
    check_pools(cache, p, slab_bytes)
    rng = random.Random(3)
    for i, op in enumerate(random_trace(rng, p, 120)):
        apply(cache, p, op)
        if i % 10 == 9:
            check_pools(cache, p, slab_bytes)
    check_pools(cache, p, slab_bytes)
    prof = tmp_path / "hot.txt"
    cache.save_profile(prof)
    assert prof.read_text() == p.profile_text()
    c2 = ops.ExpertCache(3, E, srcs, budget, n_used, copy_engine=ce)
    p2 = ExpertCachePolicy(3, E, n_used, sigs, budget)
    assert c2.load_prefetch(prof) == p2.load_prefetch(prof.read_text())
    check_pools(c2, p2, slab_bytes)
    cache.close()
    c2.close()


@pytest.mark.parametrize("tier", [1, 0])
def test_gguf_tiers_pool_bytes(tmp_path, tier):
    """The GGUF fixtures through the file tier (pread from the shard files) and
    the host tier (a pinned copy read at creation): slot bytes equal the file's."""
    sys.path.insert(0, str(ROOT / "tests"))
    import gguf_fixtures as FX
    FX.write_all(tmp_path, Oracle())
    for fname in ("moe_tiny.gguf", "moe_split-00001-of-00002.gguf"):
        note(f"gguf {'file' if tier else 'host'} tier: {fname}")
        with ops.Gguf(tmp_path / fname) as g:
            hp = g.hparams()
            n_layer, E = hp["n_layer"], hp["n_expert"]
            infos = [[g.tensor(f"blk.{l}.ffn_{nm}_exps.weight") for l in range(n_layer)]
                     for nm in ("gate", "up", "down")]
            shard_files = sorted(tmp_path.glob(fname.replace("00001", "0000?"))) if "split" in fname \
                else [tmp_path / fname]
            sigs = [[(ti["type"], ti["ne"][0], ti["ne"][1], ti["size"] // E) for ti in row] for row in infos]
            total = sum(s[3] for row in sigs for s in row) * E
            budget = int(total * 0.4)
            cache = ops.ExpertCache.from_gguf(g, tier, budget, io_threads=4)
            p = ExpertCachePolicy(n_layer, E, hp["n_expert_used"], sigs, budget)
            data = [f.read_bytes() for f in shard_files]

            def slab_bytes(r, l, e):
                ti = infos[r][l]
                n = ti["size"] // E
                off = ti["file_offset"] + e * n
                return data[ti["shard"]][off:off + n]

            rng = random.Random(11 + tier)
            for i, op in enumerate(random_trace(rng, p, 60)):
                apply(cache, p, op)
                if i % 6 == 5:
                    check_pools(cache, p, slab_bytes)
            check_pools(cache, p, slab_bytes)
            cache.close()


class CachedLayers:
    """n_layer layers of synthetic weights quantized on the GPU: all-resident
    device tensors (the reference result) and pinned host copies feeding an
    expert cache whose pools are shared by the layers (one signature)."""

    def __init__(self, n_layer, H, E, k, F, types, frac, seed):
        self.H, self.E, self.k, self.F, self.types = H, E, k, F, types
        self.resident, self.routers, self.keep, self.host = [], [], [], [[], [], []]
        tmp = torch.empty(E * F * H, dtype=torch.float32, device=DEV)
        for l in range(n_layer):
            router = torch.empty((E, H), dtype=torch.float32, device=DEV)
            ops.randn_(router, seed * 100 + l * 10 + 1, 0.0, 0.02)
            mats = []
            for j, (t, rows, cols) in enumerate(((types[0], F, H), (types[1], F, H), (types[2], H, F))):
                ops.randn_(tmp, seed * 100 + l * 10 + 2 + j, 0.0, 0.02)
                m = ops.quantize_chunk(t, tmp.view(E * rows, cols)).view(E, -1)
                mats.append(m)
                self.host[j].append(m.cpu().reshape(-1).pin_memory())
            self.routers.append(router)
            self.keep.append(mats)
            self.resident.append(ops.make_layer(H, E, k, F, router, *mats, types))
        del tmp
        torch.cuda.synchronize()
        shapes = ((H, F), (H, F), (F, H))
        srcs = [[{"type": types[r], "ne0": shapes[r][0], "ne1": shapes[r][1], "host": self.host[r][l].data_ptr()}
                 for l in range(n_layer)] for r in range(3)]
        slab = [row_size(types[r], shapes[r][0]) * shapes[r][1] for r in range(3)]
        budget = int(sum(slab) * E * n_layer * frac)
        self.cache = ops.ExpertCache(n_layer, E, srcs, budget, k)
        self.cached = []
        for l in range(n_layer):
            L = ops.make_layer(H, E, k, F, self.routers[l], *self.keep[l], types)   # shapes and router
            self.cache.layer(l, L)                                                  # pools and device rows
            self.cached.append(L)

    def resident_all(self, l, ids) -> bool:
        return all(self.cache.resident(r, l, int(e)) for e in ids for r in range(3))


def bits(t):
    return t.detach().cpu().numpy().view(np.uint32)


def test_ffn_layer_through_cache():
    note("ffn_layer through the cache: 2 layers H=1024 E=32 k=4 F=512 (Q4_K, Q4_K, Q6_K), 50% resident")
    cl = CachedLayers(2, 1024, 32, 4, 512, (Q4_K, Q4_K, Q6_K), 0.5, seed=5)
    assert cl.cache.capacity(0) == 32
    rng = np.random.default_rng(1)
    for T in (1, 3, 17, 1, 64):
        for l in range(2):
            x = torch.from_numpy(rng.standard_normal((T, 1024)).astype(np.float32)).to(DEV)
            ref_out, ref_xn, ref_ids, ref_w = ops.ffn_layer(cl.resident[l], x, rms_eps=1e-6)
            ids = sorted(set(ref_ids.cpu().numpy().reshape(-1).tolist()))
            cl.cache.ensure(l, ids)
            out, xn, got_ids, w = ops.ffn_layer(cl.cached[l], x, rms_eps=1e-6)
            torch.cuda.synchronize()
            assert torch.equal(got_ids, ref_ids), f"T={T} layer {l} ids"
            assert np.array_equal(bits(w), bits(ref_w)), f"T={T} layer {l} weights"
            assert np.array_equal(bits(out), bits(ref_out)), f"T={T} layer {l} out"
            assert np.array_equal(bits(xn), bits(ref_xn)), f"T={T} layer {l} x_next"
    st = cl.cache.stats()
    assert st["misses"] > 0 and st["evictions"] > 0
    cl.cache.close()


def test_decode_stack_through_cache():
    """Speculate on the resident set, verify, repair: every token bit-identical
    to the all-resident stack."""
    note("decode stack through the cache: 3 layers H=1024 E=16 k=4 F=512 Q4_K, 50% resident, 12 tokens")
    n_layer, H, E, k, F = 3, 1024, 16, 4, 512
    eps = 1e-6
    cl = CachedLayers(n_layer, H, E, k, F, (Q4_K,) * 3, 0.5, seed=9)
    assert cl.cache.capacity(0) >= n_layer * k
    ref_stack = ops.DecodeStack(cl.resident, eps, keepalive=cl)
    spec_stack = ops.DecodeStack(cl.cached, eps, keepalive=cl)
    rng = np.random.default_rng(2)
    n_spec_ok = n_fallback = 0
    for t in range(12):
        x = torch.from_numpy(rng.standard_normal(H).astype(np.float32)).to(DEV)
        ref_out, ref_xo, ref_ids, _ = ref_stack(x)
        out, xo, ids, _ = spec_stack(x)
        torch.cuda.synchronize()
        ids_h = ids.cpu().numpy()
        all_res = all(cl.resident_all(l, ids_h[l]) for l in range(n_layer))
        hits0 = cl.cache.stats()["hits"]
        assert (cl.cache.verify(ids_h) == 0) == all_res
        if all_res:
            # accepted: the speculative run used resident experts only (verify touched them)
            assert cl.cache.stats()["hits"] == hits0 + 3 * n_layer * k
            assert np.array_equal(bits(out), bits(ref_out)), f"token {t}: accepted speculative output"
            assert torch.equal(ids, ref_ids)
            n_spec_ok += 1
            continue
        assert cl.cache.stats()["hits"] == hits0
        # miss: per-layer path -- router, ensure, experts (decode_cached), through
        # qwmoe_expert_cache_run_layer on odd tokens and host calls on even ones
        n_fallback += 1
        xl = x.view(1, H)
        for l in range(n_layer):
            if t % 2:
                lout, xn, lid2, _ = cl.cache.run_layer(l, cl.cached[l], xl, rms_eps=eps)
            else:
                _, _, lid, _ = ops.ffn_layer(cl.cached[l], xl, rms_eps=eps)
                cl.cache.ensure(l, lid.cpu().numpy().reshape(-1).tolist())
                lout, xn, lid2, _ = ops.ffn_layer(cl.cached[l], xl, rms_eps=eps)
                assert torch.equal(lid2, lid)
            assert torch.equal(lid2.view(-1), ref_ids[l]), f"token {t} layer {l} ids"
            xl = xn
        torch.cuda.synchronize()
        assert np.array_equal(bits(lout.view(-1)), bits(ref_out)), f"token {t}: fallback output"
        assert np.array_equal(bits(xl.view(-1)), bits(ref_xo)), f"token {t}: fallback x_out"
        # everything this token needs is now resident: the speculative run verifies
        out2, _, ids2, _ = spec_stack(x)
        torch.cuda.synchronize()
        assert all(cl.resident_all(l, ids2.cpu().numpy()[l]) for l in range(n_layer))
        assert np.array_equal(bits(out2), bits(ref_out)), f"token {t}: speculative rerun"
    note(f"{n_spec_ok} tokens accepted speculatively, {n_fallback} repaired")
    assert n_fallback > 0
    assert spec_stack.status() & ~1 == 0
    spec_stack.close()
    ref_stack.close()
    cl.cache.close()


def test_file_tier_read_failure_leaves_slots_empty(tmp_path):
    """A file-tier fetch whose read fails (the file truncated under the cache,
    forced from the host) returns QWMOE_ERR_IO, leaves the unread slots absent,
    counts no fetched bytes for them, and the same call succeeds once the file
    is back."""
    sys.path.insert(0, str(ROOT / "tests"))
    import gguf_fixtures as FX
    FX.write_all(tmp_path, Oracle())
    path = tmp_path / "moe_tiny.gguf"
    good = path.read_bytes()
    note("file tier: read failure on a truncated file, then recovery")
    with ops.Gguf(path) as g:
        cache = ops.ExpertCache.from_gguf(g, 1, 10 ** 9, io_threads=2)
        cache.ensure(0, [0, 1])
        before = cache.stats()
        path.write_bytes(good[:4096])            # the data section is gone
        with pytest.raises(qa.QwmoeError) as ei:
            cache.ensure(1, [2, 3])
        assert ei.value.status == -7             # QWMOE_ERR_IO
        for r in range(3):
            for e in (2, 3):
                assert not cache.resident(r, 1, e)
            for e in (0, 1):
                assert cache.resident(r, 0, e)
        after = cache.stats()
        assert after["fetch_bytes"] == before["fetch_bytes"]
        assert after["misses"] == before["misses"] + 6
        path.write_bytes(good)
        cache.ensure(1, [2, 3])
        cache.sync()
        assert all(cache.resident(r, 1, e) for r in range(3) for e in (2, 3))
        cache.close()


def test_resident_decode_through_cache():
    """decode_cached_fast's resident mode (core/runtime.cpp:2895-3008): every
    layer's router is masked to the experts the cache holds (mask rows from
    qwmoe_expert_cache_resmask), the whole stack runs in one launch and cannot
    miss, and the unmasked top k it records (want) drives the background refill
    (qwmoe_expert_cache_refill, 8 fetches per token).  Each token's output is
    bit-identical to the all-resident weights under the same masks, every
    selected expert is resident, and the refill brings wanted experts in."""
    note("resident decode through the cache: 3 layers H=1024 E=16 k=4 F=512 Q4_K, 50% resident, 16 tokens")
    n_layer, H, E, k, F = 3, 1024, 16, 4, 512
    eps = 1e-6
    cl = CachedLayers(n_layer, H, E, k, F, (Q4_K,) * 3, 0.5, seed=13)
    mask_dev = torch.zeros((n_layer, E), dtype=torch.float32, device=DEV)
    want_dev = torch.zeros((n_layer, k), dtype=torch.int32, device=DEV)

    def masked(descs):
        out = []
        for l, L0 in enumerate(descs):
            L = qa.Layer.from_buffer_copy(L0)
            L.resmask, L.want_ids = mask_dev[l].data_ptr(), want_dev[l].data_ptr()
            out.append(L)
        return out

    stack = ops.DecodeStack(masked(cl.cached), eps, keepalive=(cl, mask_dev, want_dev))
    ref = ops.DecodeStack(masked(cl.resident), eps, keepalive=(cl, mask_dev, want_dev))
    rng = np.random.default_rng(5)
    for l in range(n_layer):   # a warm palette: 8 experts per layer (the pools' 24 slots)
        cl.cache.ensure(l, list(rng.choice(E, 8, replace=False)))
    cursor, stamp, fetched_total = 0, None, 0
    for t in range(16):
        st = cl.cache.stats()
        if (st["misses"], st["evictions"]) != stamp:      # residency changed: new mask rows
            m, complete = cl.cache.resmask(k, mask_dev)
            stamp = (st["misses"], st["evictions"])
            assert complete
            for l in range(n_layer):
                assert all((m[l, e] == 0.0) == cl.resident_all(l, [e]) for e in range(E))
        x = torch.from_numpy(rng.standard_normal(H).astype(np.float32)).to(DEV)
        r_out, r_xo, r_ids, _ = ref(x)
        out, xo, ids, _ = stack(x)
        torch.cuda.synchronize()
        assert torch.equal(ids, r_ids), f"token {t} ids"
        assert np.array_equal(bits(out), bits(r_out)), f"token {t} out"
        assert np.array_equal(bits(xo), bits(r_xo)), f"token {t} x_out"
        ids_h, want_h = ids.cpu().numpy(), want_dev.cpu().numpy()
        assert cl.cache.verify(ids_h, touch=False) == 0, f"token {t}: the masked stack picked an absent expert"
        absent = sum(not cl.resident_all(l, [e]) for l in range(n_layer) for e in want_h[l])
        fetched, cursor = cl.cache.refill(ids_h, want_h, 8, cursor)
        assert 0 <= fetched <= 8 and (absent == 0) == (fetched == 0)
        fetched_total += fetched
    note(f"refill fetched {fetched_total} experts over 16 tokens")
    assert fetched_total > 0
    assert stack.status() & ~1 == 0
    stack.close()
    ref.close()
    cl.cache.close()


def test_run_batch_slices_within_capacity():
    """The chunked prefill's layer through the cache (qwmoe_expert_cache_run_batch):
    a 200-token batch naming every expert, pools at 75 % -- the slices planned
    against capacity(layer) run one after another; outputs, ids and weights
    bit-identical to the all-resident layer on the whole batch."""
    note("run_batch: 1 layer H=1024 E=32 k=4 F=512 (Q4_K, Q4_K, Q6_K), 75% resident, T=200 and T=3")
    cl = CachedLayers(1, 1024, 32, 4, 512, (Q4_K, Q4_K, Q6_K), 0.75, seed=17)
    cap = cl.cache.capacity(0)
    rng = np.random.default_rng(9)
    for T, max_slice in ((200, 1024), (200, 16), (3, 1024)):
        x = torch.from_numpy(rng.standard_normal((T, 1024)).astype(np.float32)).to(DEV)
        ref_out, ref_xn, ref_ids, ref_w = ops.ffn_layer(cl.resident[0], x, rms_eps=1e-6)
        plan = cl.cache.plan_slices(0, ref_ids.cpu().numpy(), max_slice)
        out, xn, ids, w, ns = cl.cache.run_batch(0, cl.cached[0], x, rms_eps=1e-6, max_slice=max_slice)
        torch.cuda.synchronize()
        note(f"  T={T} max_slice={max_slice}: capacity {cap}, {ns} slices {plan[:4]}...")
        assert ns == len(plan) and (T < 20 or 1 < ns < T)
        assert torch.equal(ids, ref_ids)
        assert np.array_equal(bits(w), bits(ref_w))
        assert np.array_equal(bits(out), bits(ref_out))
        assert np.array_equal(bits(xn), bits(ref_xn))
    cl.cache.close()
