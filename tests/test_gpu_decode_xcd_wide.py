"""GPU parity of the wide form of the XCD decode kernel (qwmoe_decode_stack_*
at H = 4096, F = 1536, E = 128: the configs[4] shape, Qwen3-235B-A22B), on a
256-CU device.

Free-running stacks against the CPU oracle, bit for bit: every layer's router
ids and weights, the last layer's output and its RMSNorm; Q6_K and Q4_K down
projections, permuted slot pools, tied router logits (the exact top-k path,
std::sort replayed, blocks reloaded when the speculative expert was wrong),
k < 8 (XCDs without an expert), expert_weights_scale, resident-only masks.
The device-scope form and the layer stack at T = 1 must give the same bits.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from questwend_amd import ops  # noqa: E402
from oracle_lib import Q4_K, Q6_K, Oracle  # noqa: E402
from test_gpu_decode import GpuLayer, bits, run_and_compare  # noqa: E402

DEV = "cuda:0"
H, E, F = 4096, 128, 1536
Q6 = (Q4_K, Q4_K, Q6_K)


def note(msg: str) -> None:
    print(f"[gpu-decode-xcd-wide] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the XCD kernels need a 256-CU device")
    yield
    torch.cuda.synchronize()


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def make_stack(descs, keep, env=None):
    old = {k: os.environ.get(k) for k in (env or {})}
    os.environ.update(env or {})
    try:
        return ops.DecodeStack(descs, 1e-6, keepalive=keep)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def tokens(seed, n):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal(H).astype(np.float32) for _ in range(n)]


def test_wide_kernel_selected_q6k_down(orc):
    note("wide XCD kernel: 3 layers H=4096 E=128 k=8 F=1536 Q6_K down (layer 1 permuted), 3 tokens vs oracle")
    layers = [GpuLayer(H, E, 8, F, Q6, seed=900 + i, permute=(i == 1)) for i in range(3)]
    stack = make_stack([g.layer for g in layers], layers)
    assert stack.kernel() == 4, f"kernel {stack.kernel()} (4 expected on MI355X)"
    stack.close()
    run_and_compare(orc, layers, tokens(20, 3))


def test_wide_kernel_q4k_down(orc):
    note("wide XCD kernel: 2 layers, Q4_K down, 2 tokens vs oracle")
    layers = [GpuLayer(H, E, 8, F, (Q4_K,) * 3, seed=920 + i) for i in range(2)]
    stack = make_stack([g.layer for g in layers], layers)
    assert stack.kernel() == 4, f"kernel {stack.kernel()}"
    stack.close()
    run_and_compare(orc, layers, tokens(21, 2))


def test_wide_kernel_ties_k7(orc):
    """Router rows equal in pairs with k = 7: ties inside the first k places and
    across the k-th (the exact path; std::sort replayed; XCDs whose speculative
    expert was wrong reload their blocks); XCD 7 has no expert."""
    note("wide XCD kernel: tied router logits, k=7, 2 layers, 2 tokens vs oracle")
    layers = [GpuLayer(H, E, 7, F, Q6, seed=940 + i, dup_router=True) for i in range(2)]
    run_and_compare(orc, layers, tokens(22, 2))


def test_wide_kernel_k4_scale(orc):
    """k = 4 (four XCDs without an expert, their logits still exchanged) and
    expert_weights_scale = 2.5 (core/runtime.cpp:896-897)."""
    note("wide XCD kernel: k=4, expert_weights_scale 2.5, 2 layers, 2 tokens vs oracle")
    layers = [GpuLayer(H, E, 4, F, Q6, seed=960 + i) for i in range(2)]
    for g in layers:
        g.layer.expert_weights_scale = 2.5
        g.host.scale = 2.5
    stack = make_stack([g.layer for g in layers], layers)
    xs = tokens(23, 2)
    for t, x in enumerate(xs):
        out, xo, ids, w = stack(torch.from_numpy(x).to(DEV))
        torch.cuda.synchronize()
        xr = x.reshape(1, -1)
        for l, g in enumerate(layers):
            r = orc.moe_layer(g.host, xr, rms_eps=1e-6, scale=2.5)
            assert np.array_equal(ids.cpu().numpy()[l], r["ids"][0]), f"token {t} layer {l} ids"
            assert np.array_equal(bits(w.cpu().numpy()[l]), bits(r["weights"][0])), f"token {t} layer {l} weights"
            xr = r["xnext"]
        assert np.array_equal(bits(out.cpu().numpy()), bits(r["out"][0])), f"token {t} out"
    assert stack.status() & ~1 == 0
    stack.close()


def test_wide_kernel_device_scope_and_layer_stack_same_bits():
    """The device-scope form (kernel 5) and the layer stack at T = 1 (five
    launches per layer) give the wide kernel's bits over 4 layers x 4 tokens."""
    note("wide XCD kernel: kernel 4 vs kernel 5 vs layer stack T=1, 4 layers, 4 tokens")
    layers = [GpuLayer(H, E, 8, F, Q6, seed=980 + i, permute=(i == 2)) for i in range(4)]
    descs = [g.layer for g in layers]
    s4 = make_stack(descs, layers)
    s5 = make_stack(descs, layers, {"QWMOE_DECODE_XCD_LOCAL": "0"})
    assert (s4.kernel(), s5.kernel()) == (4, 5)
    os.environ["QWMOE_VERIFY_XCD"] = "0"   # the per-layer chain at T = 1, not the decode kernel again
    try:
        ls = ops.LayerStack(descs, 1e-6, max_tokens=1, keepalive=layers)
    finally:
        os.environ.pop("QWMOE_VERIFY_XCD", None)
    for t, x in enumerate(tokens(24, 4)):
        xd = torch.from_numpy(x).to(DEV)
        r4, r5 = s4(xd), s5(xd)
        rl = ls(xd.view(1, -1))
        torch.cuda.synchronize()
        for name, r in (("kernel 5", r5), ("layer stack", rl)):
            assert torch.equal(r4[2].view(-1), r[2].reshape(-1)), f"token {t} {name} ids"
            assert torch.equal(r4[3].view(-1).view(torch.int32), r[3].reshape(-1).view(torch.int32)), f"token {t} {name} w"
            assert torch.equal(r4[0].view(-1).view(torch.int32), r[0].reshape(-1).view(torch.int32)), f"token {t} {name} out"
            assert torch.equal(r4[1].view(-1).view(torch.int32), r[1].reshape(-1).view(torch.int32)), f"token {t} {name} x"
    assert s4.status() & ~1 == 0 and s5.status() & ~1 == 0
    s4.close()
    s5.close()
    ls.close()


def test_wide_kernel_resident_masks(orc):
    """Resident-only routing (core/runtime.cpp:870-881) through the wide kernel:
    per layer want, ids, weights and the last layer's output against the oracle
    chain, masks of 9 and 60 resident experts."""
    from test_gpu_resident import chain_oracle, masked_layers
    note("wide XCD kernel: resident masks (9, 60 of 128), 2 layers, 2 tokens vs oracle")
    layers = [GpuLayer(H, E, 8, F, Q6, seed=1000 + i) for i in range(2)]
    descs, masks, wants, keep = masked_layers(layers, [9, 60], seed=9)
    stack = make_stack(descs, keep)
    assert stack.kernel() == 4
    for t, x in enumerate(tokens(25, 2)):
        out, xo, ids, w = stack(torch.from_numpy(x).to(DEV))
        torch.cuda.synchronize()
        rs = chain_oracle(orc, layers, masks, x.reshape(1, -1))
        for l, r in enumerate(rs):
            assert np.array_equal(wants[l].cpu().numpy()[0], r["want"][0]), f"token {t} layer {l} want"
            assert np.array_equal(ids.cpu().numpy()[l], r["ids"][0]), f"token {t} layer {l} ids"
            assert np.array_equal(bits(w.cpu().numpy()[l]), bits(r["weights"][0])), f"token {t} layer {l} weights"
        assert np.array_equal(bits(out.cpu().numpy()), bits(rs[-1]["out"][0])), f"token {t} out"
    assert stack.status() & ~1 == 0
    stack.close()
