"""GPU parity of the persistent verify-batch kernel (verify_xcd.hip), the path
qwmoe_layer_stack_run takes for 2 <= T <= 8 tokens at the Qwen3-30B-A3B shape
(H = 2048, F = 768, Q4_K) on a 256-CU device: one launch for all layers, the
batch's distinct experts dealt to the XCDs.

Free-running stacks against the CPU oracle's T-token layers (build_moe's T > 1
mul + add-chain weighted sum), bit for bit: every layer's ids and weights, the
last layer's output and its RMSNorm; T = 2..8, permuted slot pools, tied router
logits (the exact top-k per token, std::sort replayed), k = 4 with
expert_weights_scale, E = 32; and the same bits as the per-layer chain
(QWMOE_VERIFY_XCD=0) over 8 layers.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from questwend_amd import ops  # noqa: E402
from oracle_lib import Q4_K, Oracle  # noqa: E402
from test_gpu_decode import GpuLayer, bits  # noqa: E402

DEV = "cuda:0"
H, F = 2048, 768


def note(msg: str) -> None:
    print(f"[gpu-verify-xcd] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the persistent verify kernel needs a 256-CU device")
    prev = ops.set_mfma_form(ops.MFMA_EXACT)   # the per-layer chain compared against it: bit-exact form
    yield
    torch.cuda.synchronize()
    ops.set_mfma_form(prev)


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def make_stack(layers, max_tokens=8, env=None):
    old = {k: os.environ.get(k) for k in (env or {})}
    os.environ.update(env or {})
    try:
        return ops.LayerStack([g.layer for g in layers], 1e-6, max_tokens=max_tokens, keepalive=layers)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def check_vs_oracle(orc, stack, layers, x, scale=None, what=""):
    T = x.shape[0]
    out, xo, ids, w = stack(torch.from_numpy(x).to(DEV))
    torch.cuda.synchronize()
    xr = x
    kw = {} if scale is None else {"scale": scale}
    for l, g in enumerate(layers):
        r = orc.moe_layer(g.host, xr, rms_eps=1e-6, **kw)
        assert np.array_equal(ids[l].cpu().numpy(), r["ids"]), f"{what} T={T} layer {l} ids"
        assert np.array_equal(bits(w[l].cpu().numpy()), bits(r["weights"])), f"{what} T={T} layer {l} weights"
        xr = r["xnext"]
    assert np.array_equal(bits(out.cpu().numpy()), bits(r["out"])), f"{what} T={T} out"
    assert np.array_equal(bits(xo.cpu().numpy()), bits(r["xnext"])), f"{what} T={T} x_out"


def test_verify_kernel_t2_to_t8(orc):
    note("verify kernel: 3 layers H=2048 E=128 k=8 F=768 (layer 1 permuted), T = 2..8 vs oracle")
    layers = [GpuLayer(H, 128, 8, F, (Q4_K,) * 3, seed=1100 + i, permute=(i == 1)) for i in range(3)]
    stack = make_stack(layers)
    assert stack.kernel() == 2, f"kernel {stack.kernel()} (2 expected on MI355X)"
    rng = np.random.default_rng(30)
    for T in (2, 3, 5, 8, 4, 6, 7):
        c = rng.standard_normal(H)
        x = (np.sqrt(0.8) * c + np.sqrt(0.2) * rng.standard_normal((T, H))).astype(np.float32)   # overlapping experts
        check_vs_oracle(orc, stack, layers, x)
        x = rng.standard_normal((T, H)).astype(np.float32)                                     # mostly distinct
        check_vs_oracle(orc, stack, layers, x)
    assert stack.status() & ~1 == 0
    stack.close()


def test_verify_kernel_ties(orc):
    """Router rows equal in pairs: ties inside and across every token's first k
    places (each token's wave takes the exact path and replays std::sort)."""
    note("verify kernel: tied router logits, 2 layers E=128 k=7, T = 3, 6 vs oracle")
    layers = [GpuLayer(H, 128, 7, F, (Q4_K,) * 3, seed=1120 + i, dup_router=True) for i in range(2)]
    stack = make_stack(layers)
    assert stack.kernel() == 2
    rng = np.random.default_rng(31)
    for T in (3, 6):
        check_vs_oracle(orc, stack, layers, rng.standard_normal((T, H)).astype(np.float32), what="ties")
    assert stack.status() & 1, "the ties reached the std::sort replay"
    stack.close()


def test_verify_kernel_k4_scale_e32(orc):
    """E = 32 (one logit per router wave's half) with k = 4 and
    expert_weights_scale = 2.5 (core/runtime.cpp:896-897)."""
    note("verify kernel: E=32 k=4 expert_weights_scale 2.5, 2 layers, T = 2, 5, 8 vs oracle")
    layers = [GpuLayer(H, 32, 4, F, (Q4_K,) * 3, seed=1140 + i) for i in range(2)]
    for g in layers:
        g.layer.expert_weights_scale = 2.5
        g.host.scale = 2.5
    stack = make_stack(layers)
    assert stack.kernel() == 2
    rng = np.random.default_rng(32)
    for T in (2, 5, 8):
        check_vs_oracle(orc, stack, layers, rng.standard_normal((T, H)).astype(np.float32), scale=2.5, what="scale")
    assert stack.status() & ~1 == 0
    stack.close()


def test_verify_kernel_equals_per_layer_chain():
    """8 layers of the 30B shape, T = 5 correlated tokens, 6 steps: the
    persistent kernel (XCD-local and device-scope words) and the per-layer chain
    give the same bits, and at T = 1 the stack (on the decode kernel) equals the chain."""
    note("verify kernel vs device-scope form vs per-layer chain: 8 layers, T=5, 6 steps")
    layers = [GpuLayer(H, 128, 8, F, (Q4_K,) * 3, seed=1160 + i, permute=(i % 3 == 0)) for i in range(8)]
    s2 = make_stack(layers)
    s3 = make_stack(layers, env={"QWMOE_DECODE_XCD_LOCAL": "0"})
    s1 = make_stack(layers, env={"QWMOE_VERIFY_XCD": "0"})
    assert (s2.kernel(), s3.kernel(), s1.kernel()) == (2, 3, 1)
    rng = np.random.default_rng(33)
    for step in range(6):
        c = rng.standard_normal(H)
        x = (np.sqrt(0.8) * c + np.sqrt(0.2) * rng.standard_normal((5, H))).astype(np.float32)
        xd = torch.from_numpy(x).to(DEV)
        r2, r3, r1 = s2(xd), s3(xd), s1(xd)
        torch.cuda.synchronize()
        for name, r in (("device scope", r3), ("per-layer chain", r1)):
            assert torch.equal(r2[2], r[2]), f"step {step} {name} ids"
            for a_, b_, what in ((r2[3], r[3], "weights"), (r2[0], r[0], "out"), (r2[1], r[1], "x_out")):
                assert torch.equal(a_.view(torch.int32), b_.view(torch.int32)), f"step {step} {name} {what}"
    x1 = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to(DEV)
    a1, b1 = s2(x1), s1(x1)
    torch.cuda.synchronize()
    assert torch.equal(a1[0].view(torch.int32), b1[0].view(torch.int32))
    assert s2.status() & ~1 == 0 and s3.status() & ~1 == 0
    for s in (s1, s2, s3):
        s.close()
