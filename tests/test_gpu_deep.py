"""Parity at the configured depths and lengths, against the reference's own
ggml (oracle/_ref/libqwref.so, AVX2 branch; tests/test_oracle.py pins the
restatement to it bit for bit), free-running: every layer takes the previous
layer's RMSNorm output as the GPU computed it.

  configs[1]  48 Q4_K layers of the 30B-A3B shape, 256 decode steps (+8 warm-up)
              through the persistent decode stack: every layer's ids of every
              step and every step's output, bit for bit.
  configs[3]  1000 seeded verify batches (T = 5, tokens correlated at rho = 0.8)
              through one 30B-A3B Q4_K layer: ids, weights, output, RMSNorm.
  configs[4]  94 layers at H = 4096, E = 128, F = 1536 (Q4_K gate/up, Q6_K
              down) through the layer stack's captured graph at T = 1 and
              through the persistent decode kernel, every layer read through a
              seeded slot permutation.  The routers are
              distinct per layer; the expert tensors come from 4 distinct sets,
              layer l using set l % 4 (all 94 distinct would need 147 GB).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from questwend_amd import ops, row_size  # noqa: E402
from oracle_lib import Q4_K, Q6_K, LayerWeights, RefGGML, have_ref  # noqa: E402

DEV = "cuda:0"
EPS = 1e-6


def note(msg: str) -> None:
    print(f"[gpu-deep] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not have_ref():
        pytest.skip("oracle/_ref/libqwref.so not built (needs the reference tree at build time)")
    ops.init(0, 1 << 30)
    prev = ops.set_mfma_form(ops.MFMA_EXACT)
    yield
    torch.cuda.synchronize()
    ops.set_mfma_form(prev)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.int32)


def n_threads() -> int:
    import os
    return max(1, min(16, len(os.sched_getaffinity(0))))


def gpu_mats(E, H, F, types, seed, chunk=16):
    """gate / up / down of E experts generated (N(0, 0.02)) and quantized on the GPU."""
    mats = []
    tmp = torch.empty(chunk * F * H, dtype=torch.float32, device=DEV)
    for j, (t, rows, cols) in enumerate(((types[0], F, H), (types[1], F, H), (types[2], H, F))):
        q = torch.empty((E * rows, row_size(t, cols)), dtype=torch.uint8, device=DEV)
        for e0 in range(0, E, chunk):
            n = chunk * rows * cols
            ops.randn_(tmp[:n], seed * 1000 + j * 100 + e0, 0.0, 0.02)
            ops.quantize_chunk_into(t, tmp[:n].view(chunk * rows, cols), q[e0 * rows:(e0 + chunk) * rows])
        mats.append(q.view(E, -1))
    del tmp
    return mats


def host_layer(H, E, k, F, types, router, mats) -> LayerWeights:
    lw = LayerWeights.__new__(LayerWeights)
    lw.H, lw.E, lw.k, lw.F = H, E, k, F
    lw.type_gate, lw.type_up, lw.type_down = types
    lw.router = router.cpu().numpy()
    lw.gate, lw.up, lw.down = (m.cpu().numpy().reshape(-1) for m in mats)
    lw.n_slots, lw.slot_of = E, None
    return lw


def test_config1_48_layers_256_steps():
    H, E, k, F, NL = 2048, 128, 8, 768, 48
    steps, warm = 256, 8
    note(f"configs[1]: {NL} layers, {steps} steps + {warm} warm-up, decode stack vs ggml (AVX2)")
    types = (Q4_K,) * 3
    layers, keep, lws = [], [], []
    for l in range(NL):
        router = torch.empty((E, H), dtype=torch.float32, device=DEV)
        ops.randn_(router, 5000 + l, 0.0, 0.02)
        mats = gpu_mats(E, H, F, types, seed=5100 + l)
        layers.append(ops.make_layer(H, E, k, F, router, *mats, types))
        keep.append((router, mats))
        lws.append(host_layer(H, E, k, F, types, router, mats))
    xs = np.random.default_rng(77).standard_normal((warm + steps, H)).astype(np.float32)
    stack = ops.DecodeStack(layers, EPS, keepalive=keep)
    xd = torch.from_numpy(xs).to(DEV)
    g_out = np.zeros((steps, H), np.float32)
    g_ids = np.zeros((steps, NL, k), np.int32)
    for s in range(warm + steps):
        out, _, ids, _ = stack(xd[s])
        if s >= warm:
            g_out[s - warm] = out.cpu().numpy()
            g_ids[s - warm] = ids.cpu().numpy()
    assert stack.status() & ~1 == 0
    stack.close()
    ref = RefGGML()
    RL = [ref.layer(lw, 1, rms_eps=EPS, n_threads=n_threads()) for lw in lws]
    r = ref.stack_run(RL, xs, warm, n_threads())
    first = next((s for s in range(steps) if not np.array_equal(g_ids[s], r["ids"][s])), None)
    note(f"  ids equal on {sum(np.array_equal(g_ids[s], r['ids'][s]) for s in range(steps))}/{steps} steps; "
         f"smallest top-k margin {float(r['margin'].min()):.3e}")
    assert first is None, f"step {first}: ids differ at layer {np.nonzero((g_ids[first] != r['ids'][first]).any(1))[0]}"
    assert np.array_equal(bits(g_out), bits(r["out"]))


def test_config3_1000_verify_batches():
    H, E, k, F = 2048, 128, 8, 768
    note("configs[3]: 1000 T=5 correlated verify batches through a 30B-A3B Q4_K layer vs ggml (AVX2)")
    types = (Q4_K,) * 3
    router = torch.empty((E, H), dtype=torch.float32, device=DEV)
    ops.randn_(router, 6001, 0.0, 0.02)
    mats = gpu_mats(E, H, F, types, seed=6100)
    L = ops.make_layer(H, E, k, F, router, *mats, types)
    lw = host_layer(H, E, k, F, types, router, mats)
    RL = RefGGML().layer(lw, 5, rms_eps=EPS, n_threads=n_threads())
    stack = ops.LayerStack([L], EPS, max_tokens=5, keepalive=(router, mats))
    rng = np.random.default_rng(3)
    distinct = []
    for step in range(1000):
        c = rng.standard_normal(H)
        x = (np.sqrt(0.8) * c + np.sqrt(0.2) * rng.standard_normal((5, H))).astype(np.float32)
        out, xn, ids, w = stack(torch.from_numpy(x).to(DEV))
        r = RL(x)
        ids_h = ids.cpu().numpy()[0]
        assert np.array_equal(ids_h, r["ids"]), f"step {step} ids"
        assert np.array_equal(bits(w.cpu().numpy()[0]), bits(r["weights"])), f"step {step} weights"
        assert np.array_equal(bits(out.cpu().numpy()), bits(r["out"])), f"step {step} out"
        assert np.array_equal(bits(xn.cpu().numpy()), bits(r["xnext"])), f"step {step} x_next"
        distinct.append(len(np.unique(ids_h)))
    note(f"  distinct experts per batch: mean {np.mean(distinct):.1f} of 40 selections")
    assert np.mean(distinct) < 40
    stack.close()


def test_config4_94_layers_slot_tables():
    H, E, k, F, NL, NSET = 4096, 128, 8, 1536, 94, 4
    steps, warm = 6, 2
    types = (Q4_K, Q4_K, Q6_K)
    note(f"configs[4]: {NL} layers (expert sets: {NSET}), permuted slots, layer stack T=1, {steps} steps vs ggml")
    g = torch.Generator().manual_seed(40)
    sets, pools, slots, host_sets = [], [], [], []
    for sidx in range(NSET):
        mats = gpu_mats(E, H, F, types, seed=7000 + sidx)
        perm = [torch.randperm(E, generator=g).to(torch.int32) for _ in range(3)]
        pl = []
        for m, p in zip(mats, perm):
            pool = torch.empty_like(m)
            pool[p.long().to(DEV)] = m                 # logical expert e at slot p[e]
            pl.append(pool)
        host_sets.append(tuple(m.cpu().numpy().reshape(-1) for m in mats))
        pools.append(pl)
        slots.append(tuple(p.to(DEV) for p in perm))
        del mats
    layers, keep, lws = [], [pools, slots], []
    for l in range(NL):
        router = torch.empty((E, H), dtype=torch.float32, device=DEV)
        ops.randn_(router, 7100 + l, 0.0, 0.02)
        sidx = l % NSET
        layers.append(ops.make_layer(H, E, k, F, router, *pools[sidx], types, n_slots=(E, E, E), slots=slots[sidx]))
        keep.append(router)
        lw = LayerWeights.__new__(LayerWeights)
        lw.H, lw.E, lw.k, lw.F = H, E, k, F
        lw.type_gate, lw.type_up, lw.type_down = types
        lw.router = router.cpu().numpy()
        lw.gate, lw.up, lw.down = host_sets[sidx]
        lw.n_slots, lw.slot_of = E, None
        lws.append(lw)
    xs = np.random.default_rng(94).standard_normal((warm + steps, H)).astype(np.float32)
    xd = torch.from_numpy(xs).to(DEV)
    runs = {}
    # the layer stack (five launches per layer) and the persistent decode kernel
    # (one launch per token; its wide XCD form on a 256-CU device)
    for name in ("layer stack", "decode stack"):
        if name == "layer stack":
            os.environ["QWMOE_VERIFY_XCD"] = "0"   # the per-layer chain (T = 1 otherwise runs on the decode kernel)
            try:
                stack = ops.LayerStack(layers, EPS, max_tokens=1, keepalive=keep)
            finally:
                os.environ.pop("QWMOE_VERIFY_XCD", None)
        else:
            stack = ops.DecodeStack(layers, EPS, keepalive=keep)
            note(f"  decode stack kernel {stack.kernel()}")
        g_out, g_ids = [], []
        for s in range(warm + steps):
            out, _, ids, _ = stack(xd[s:s + 1] if name == "layer stack" else xd[s])
            if s >= warm:
                g_out.append(out.cpu().numpy().reshape(-1))
                g_ids.append(ids.cpu().numpy().reshape(NL, k))
        if name == "decode stack":
            assert stack.status() & ~1 == 0
        stack.close()
        runs[name] = (g_out, g_ids)
    ref = RefGGML()
    RL = [ref.layer(lw, 1, rms_eps=EPS, n_threads=n_threads()) for lw in lws]
    r = ref.stack_run(RL, xs, warm, n_threads())
    for name, (g_out, g_ids) in runs.items():
        for s in range(steps):
            assert np.array_equal(g_ids[s], r["ids"][s]), f"{name}: step {s} ids"
            assert np.array_equal(bits(g_out[s]), bits(r["out"][s])), f"{name}: step {s} out"
    note(f"  {steps} steps x {NL} layers equal (layer stack and decode stack); "
         f"smallest top-k margin {float(r['margin'].min()):.3e}")
