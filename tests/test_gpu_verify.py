"""GPU parity of T-token batches through a layer stack (qwmoe_layer_stack_*),
the FFN half of speculative decoding's verify forward (core/runtime.cpp:1495-1562).

* T = 1..4 tokens through three layers, free-running (RMSNorm between layers):
  every layer's ids and weights, the last layer's output and its RMSNorm equal
  the CPU oracle's T-token layers bit for bit (T > 1 takes build_moe's
  mul + add-chain weighted sum).
* The captured graph, replayed many times with changing inputs and T, eager
  library work and synchronisations in between, equals the eager chain on
  every replay.
* At T = 1 the stack equals the persistent decode stack bit for bit.
* configs[3] (5 correlated verify tokens through a 30B-A3B Q4_K layer at E = 128,
  40 seeded steps) and configs[0] (a Q8_0 layer at E = 128, decode) at their
  full shapes, against the oracle.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from questwend_amd import ops  # noqa: E402
from oracle_lib import Q4_K, Q6_K, Oracle  # noqa: E402
from test_gpu_decode import GpuLayer, bits  # noqa: E402

DEV = "cuda:0"


def note(msg: str) -> None:
    print(f"[gpu-verify] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    prev = ops.set_mfma_form(ops.MFMA_EXACT)   # bit-exact tests: the matrix cores (T >= 8 bins) replay ggml's float steps
    yield
    torch.cuda.synchronize()
    ops.set_mfma_form(prev)


@pytest.fixture(scope="module")
def orc():
    return Oracle()


@pytest.fixture(scope="module")
def layers3():
    return [GpuLayer(1024, 16, 4, 512, (Q4_K, Q4_K, Q6_K), seed=700 + i) for i in range(3)]


@pytest.mark.parametrize("graphs", [True, False])
def test_layer_stack_matches_oracle(orc, layers3, graphs):
    note(f"layer stack (graphs={graphs}): 3 layers H=1024 E=16 k=4 F=512, T = 1..4")
    stack = ops.LayerStack([g.layer for g in layers3], 1e-6, max_tokens=4, graphs=graphs, keepalive=layers3)
    rng = np.random.default_rng(5)
    for T in (1, 2, 3, 4, 2):
        x = rng.standard_normal((T, 1024)).astype(np.float32)
        out, xo, ids, w = stack(torch.from_numpy(x).to(DEV))
        torch.cuda.synchronize()
        xr = x
        for l, g in enumerate(layers3):
            r = orc.moe_layer(g.host, xr, rms_eps=1e-6)
            assert np.array_equal(ids[l].cpu().numpy(), r["ids"]), f"T={T} layer {l} ids"
            assert np.array_equal(bits(w[l].cpu().numpy()), bits(r["weights"])), f"T={T} layer {l} weights"
            xr = r["xnext"]
        assert np.array_equal(bits(out.cpu().numpy()), bits(r["out"])), f"T={T} out"
        assert np.array_equal(bits(xo.cpu().numpy()), bits(r["xnext"])), f"T={T} x_out"
    stack.close()


def test_layer_stack_graph_replays_equal_eager(layers3):
    note("layer stack: 24 graph replays (T varies) against the eager chain, eager work in between")
    Ls = [g.layer for g in layers3]
    gstack = ops.LayerStack(Ls, 1e-6, max_tokens=4, graphs=True, keepalive=layers3)
    estack = ops.LayerStack(Ls, 1e-6, max_tokens=4, graphs=False, keepalive=layers3)
    rng = np.random.default_rng(9)
    for i in range(24):
        T = (1, 3, 4, 2)[i % 4]
        x = torch.from_numpy(rng.standard_normal((T, 1024)).astype(np.float32)).to(DEV)
        go, gxo, gids, gw = gstack(x)
        if i % 3 == 0:
            torch.cuda.synchronize()
        # unrelated eager library work on the same stream and workspace
        ops.ffn_layer(Ls[i % 3], torch.from_numpy(rng.standard_normal((5, 1024)).astype(np.float32)).to(DEV),
                      rms_eps=1e-6)
        eo, exo, eids, ew = estack(x)
        torch.cuda.synchronize()
        assert torch.equal(gids, eids), f"replay {i} (T={T}) ids"
        assert torch.equal(go.view(torch.int32), eo.view(torch.int32)), f"replay {i} (T={T}) out"
        assert torch.equal(gxo.view(torch.int32), exo.view(torch.int32)), f"replay {i} (T={T}) x_out"
        assert torch.equal(gw.view(torch.int32), ew.view(torch.int32)), f"replay {i} (T={T}) weights"
    gstack.close()
    estack.close()


def test_layer_stack_t1_equals_decode_stack():
    note("layer stack T=1 vs decode stack: 2 layers of the 30B shape (H=2048 E=128 k=8 F=768 Q4_K)")
    layers = [GpuLayer(2048, 128, 8, 768, (Q4_K,) * 3, seed=800 + i) for i in range(2)]
    Ls = [g.layer for g in layers]
    os.environ["QWMOE_VERIFY_XCD"] = "0"   # the per-layer chain at T = 1 (the default hands T = 1 to the decode stack)
    try:
        stack = ops.LayerStack(Ls, 1e-6, max_tokens=1, keepalive=layers)
    finally:
        os.environ.pop("QWMOE_VERIFY_XCD", None)
    dstack = ops.DecodeStack(Ls, 1e-6, keepalive=layers)
    rng = np.random.default_rng(3)
    for t in range(4):
        x = torch.from_numpy(rng.standard_normal(2048).astype(np.float32)).to(DEV)
        out, xo, ids, w = stack(x.view(1, -1))
        dout, dxo, dids, dw = dstack(x)
        torch.cuda.synchronize()
        assert torch.equal(ids[:, 0], dids), f"token {t} ids"
        assert torch.equal(out[0].view(torch.int32), dout.view(torch.int32)), f"token {t} out"
        assert torch.equal(xo[0].view(torch.int32), dxo.view(torch.int32)), f"token {t} x_out"
        assert torch.equal(w[:, 0].view(torch.int32), dw.view(torch.int32)), f"token {t} weights"
    assert dstack.status() & ~1 == 0
    stack.close()
    dstack.close()


def correlated_tokens(rng, T, H, rho):
    """T rows of N(0, 1) with pairwise correlation rho (a shared component)."""
    c = rng.standard_normal(H)
    return (np.sqrt(rho) * c + np.sqrt(1.0 - rho) * rng.standard_normal((T, H))).astype(np.float32)


def test_config4_verify_batches_e128(orc):
    """5 tokens (1 accepted + 4 draft), activations correlated at
    rho = 0.8, through a Qwen3-30B-A3B-shaped Q4_K layer (E = 128): ids,
    weights, output and its RMSNorm equal the oracle on 40 seeded steps, through
    qwmoe_ffn_layer and through a one-layer stack's captured graph."""
    note("configs[3]: T=5 correlated verify batches, 30B-A3B Q4_K layer at E=128, 40 steps")
    g = GpuLayer(2048, 128, 8, 768, (Q4_K,) * 3, seed=900)
    stack = ops.LayerStack([g.layer], 1e-6, max_tokens=5, keepalive=g)
    rng = np.random.default_rng(4)
    overlap = []
    for step in range(40):
        x = correlated_tokens(rng, 5, 2048, 0.8)
        r = orc.moe_layer(g.host, x, rms_eps=1e-6)
        out, xn, ids, w = ops.ffn_layer(g.layer, torch.from_numpy(x).to(DEV), rms_eps=1e-6)
        so, sxo, sids, sw = stack(torch.from_numpy(x).to(DEV))
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy(), r["ids"]), f"step {step} ids"
        assert np.array_equal(bits(w.cpu().numpy()), bits(r["weights"])), f"step {step} weights"
        assert np.array_equal(bits(out.cpu().numpy()), bits(r["out"])), f"step {step} out"
        assert np.array_equal(bits(xn.cpu().numpy()), bits(r["xnext"])), f"step {step} x_next"
        assert torch.equal(sids[0], ids) and torch.equal(so.view(torch.int32), out.view(torch.int32))
        assert torch.equal(sxo.view(torch.int32), xn.view(torch.int32))
        overlap.append(len(np.unique(r["ids"])))
    note(f"distinct experts per 5-token batch: mean {np.mean(overlap):.1f} of 40 selections")
    assert np.mean(overlap) < 40          # correlated tokens share experts
    stack.close()


def test_config0_q8_0_decode_e128(orc):
    """one Qwen3-MoE FFN layer, 1-token decode, Q8_0 experts at the
    full shape (H=2048, E=128, k=8, F=768): equal to the oracle on 8 tokens."""
    note("configs[0]: Q8_0 layer at E=128, T=1, 8 tokens")
    from oracle_lib import Q8_0
    g = GpuLayer(2048, 128, 8, 768, (Q8_0,) * 3, seed=910)
    rng = np.random.default_rng(8)
    for t in range(8):
        x = rng.standard_normal((1, 2048)).astype(np.float32)
        r = orc.moe_layer(g.host, x, rms_eps=1e-6)
        out, xn, ids, w = ops.ffn_layer(g.layer, torch.from_numpy(x).to(DEV), rms_eps=1e-6)
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy(), r["ids"]), f"token {t} ids"
        assert np.array_equal(bits(w.cpu().numpy()), bits(r["weights"])), f"token {t} weights"
        assert np.array_equal(bits(out.cpu().numpy()), bits(r["out"])), f"token {t} out"
        assert np.array_equal(bits(xn.cpu().numpy()), bits(r["xnext"])), f"token {t} x_next"


@pytest.mark.parametrize("T", [1, 3, 16])
def test_small_batch_router_ties(orc, T):
    """Small batches take the router's top-k and the grouping in one launch (a
    wave per token); with router rows duplicated in pairs every top-k has ties,
    which the std::sort replay inside that launch must order as ggml does."""
    note(f"small-batch router ties: T={T}, H=1024 E=16 k=4 F=512")
    g = GpuLayer(1024, 16, 4, 512, (Q4_K,) * 3, seed=950 + T, dup_router=True)
    x = np.random.default_rng(T).standard_normal((T, 1024)).astype(np.float32)
    ops.device_status(clear=True)
    out, xn, ids, w = ops.ffn_layer(g.layer, torch.from_numpy(x).to(DEV), rms_eps=1e-6)
    torch.cuda.synchronize()
    r = orc.moe_layer(g.host, x, rms_eps=1e-6)
    assert np.array_equal(ids.cpu().numpy(), r["ids"])
    assert np.array_equal(bits(w.cpu().numpy()), bits(r["weights"]))
    assert np.array_equal(bits(out.cpu().numpy()), bits(r["out"]))
    assert np.array_equal(bits(xn.cpu().numpy()), bits(r["xnext"]))
    assert ops.device_status(clear=True) & 1      # the replay ran


def test_layer_stack_recaptures_after_workspace_realloc(layers3):
    """A captured graph holds the library workspace's addresses; after qwmoe_init
    reallocates the workspace the next run captures again and gives the same
    result."""
    note("layer stack: graph re-captured after the workspace is reallocated")
    stack = ops.LayerStack([g.layer for g in layers3], 1e-6, max_tokens=4, keepalive=layers3)
    x = torch.from_numpy(np.random.default_rng(21).standard_normal((3, 1024)).astype(np.float32)).to(DEV)
    o1, xo1, ids1, _ = stack(x)
    torch.cuda.synchronize()
    ops.init(0, 640 << 20)              # a larger workspace: freed and allocated again
    o2, xo2, ids2, _ = stack(x)
    torch.cuda.synchronize()
    assert torch.equal(ids1, ids2)
    assert torch.equal(o1.view(torch.int32), o2.view(torch.int32))
    assert torch.equal(xo1.view(torch.int32), xo2.view(torch.int32))
    stack.close()


def test_layer_stack_recaptures_after_threshold_change(layers3):
    """A captured graph holds the kernel choice the matrix-core threshold made:
    setting another threshold makes the next run capture again (same bits);
    setting the same one does not.  The threshold outlives re-initialisation."""
    note("layer stack: graph re-captured after qwmoe_set_mfma_min_rows changes the threshold")
    stack = ops.LayerStack([g.layer for g in layers3], 1e-6, max_tokens=4, keepalive=layers3)
    x = torch.from_numpy(np.random.default_rng(22).standard_normal((3, 1024)).astype(np.float32)).to(DEV)
    prev = ops.set_mfma_min_rows(2)
    try:
        o1, _, ids1, _ = stack(x)
        o1b, _, _, _ = stack(x)
        torch.cuda.synchronize()
        assert stack.captures() == 1
        ops.set_mfma_min_rows(2)                       # unchanged: the graph stays
        stack(x)
        assert stack.captures() == 1
        ops.set_mfma_min_rows(0)                       # every expert on the GEMV now
        o2, _, ids2, _ = stack(x)
        torch.cuda.synchronize()
        assert stack.captures() == 2
        assert torch.equal(ids1, ids2)
        assert torch.equal(o1.view(torch.int32), o2.view(torch.int32))
        assert torch.equal(o1.view(torch.int32), o1b.view(torch.int32))
        ops.set_mfma_min_rows(5)
        ops.init(0, 768 << 20)                         # reallocates the workspace
        assert ops.set_mfma_min_rows(5) == 5           # (returns the previous value)
    finally:
        ops.set_mfma_min_rows(prev)
    stack.close()

