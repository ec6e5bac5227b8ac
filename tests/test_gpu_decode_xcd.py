"""GPU parity of the decode kernel with one selected expert per XCD
(qwmoe_decode_stack_* on a 256-CU device at H = 2048, k <= 8, Q4_K).

Free-running stacks against the CPU oracle, bit for bit: every layer's router
ids and weights, the last layer's output and its RMSNorm.  The same stack under
the other kernel choices (device-scope exchange words; the per-CU kernel) must
give the same bits.  Weights are generated and quantized on the GPU (the
quantizer is pinned byte for byte in test_gpu_parity.py) and copied to the host
for the oracle.
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
from test_gpu_decode import GpuLayer, bits, run_and_compare  # noqa: E402

DEV = "cuda:0"
H, F = 2048, 768


def note(msg: str) -> None:
    print(f"[gpu-decode-xcd] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the XCD kernel needs a 256-CU device")
    yield
    torch.cuda.synchronize()


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def make_stack(layers, env=None):
    old = {k: os.environ.get(k) for k in (env or {})}
    os.environ.update(env or {})
    try:
        return ops.DecodeStack([g.layer for g in layers], 1e-6, keepalive=layers)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def run_tokens(stack, xs):
    outs = []
    for x in xs:
        out, xo, ids, w = stack(x)
        torch.cuda.synchronize()
        outs.append((out.clone(), xo.clone(), ids.clone(), w.clone()))
    return outs


def same_bits(a, b):
    for (o1, x1, i1, w1), (o2, x2, i2, w2) in zip(a, b):
        assert torch.equal(i1, i2)
        assert torch.equal(w1.view(torch.int32), w2.view(torch.int32))
        assert torch.equal(o1.view(torch.int32), o2.view(torch.int32))
        assert torch.equal(x1.view(torch.int32), x2.view(torch.int32))


def test_xcd_kernel_e32_three_layers(orc):
    note("XCD kernel: 3 layers H=2048 E=32 k=8 F=768, 3 tokens vs oracle")
    layers = [GpuLayer(H, 32, 8, F, (Q4_K,) * 3, seed=800 + i) for i in range(3)]
    stack = make_stack(layers)
    assert stack.kernel() in (2, 3), f"kernel {stack.kernel()}"
    stack.close()
    rng = np.random.default_rng(10)
    run_and_compare(orc, layers, [rng.standard_normal(H).astype(np.float32) for _ in range(3)])


def test_xcd_kernel_30b_shape_selected(orc):
    note("XCD kernel: 2 layers of the 30B-A3B shape (E=128), 2 tokens vs oracle")
    layers = [GpuLayer(H, 128, 8, F, (Q4_K,) * 3, seed=820 + i) for i in range(2)]
    stack = make_stack(layers)
    assert stack.kernel() == 2, f"kernel {stack.kernel()} (2 expected on MI355X)"
    stack.close()
    rng = np.random.default_rng(11)
    run_and_compare(orc, layers, [rng.standard_normal(H).astype(np.float32) for _ in range(2)])


def test_xcd_kernel_permuted_slots(orc):
    note("XCD kernel: permuted slot pools, 2 layers E=64, 2 tokens vs oracle")
    layers = [GpuLayer(H, 64, 8, F, (Q4_K,) * 3, seed=840 + i, permute=True) for i in range(2)]
    rng = np.random.default_rng(12)
    run_and_compare(orc, layers, [rng.standard_normal(H).astype(np.float32) for _ in range(2)])


def test_xcd_kernel_ties_k7(orc):
    """Router rows equal in pairs with k = 7: ties inside the first k places and
    across the k-th, so the speculative expert of some XCDs is wrong and the
    std::sort replay decides; XCD 7 has no expert."""
    note("XCD kernel: tied router logits, k=7, 3 layers E=32, 2 tokens vs oracle")
    layers = [GpuLayer(H, 32, 7, F, (Q4_K,) * 3, seed=860 + i, dup_router=True) for i in range(3)]
    rng = np.random.default_rng(13)
    run_and_compare(orc, layers, [rng.standard_normal(H).astype(np.float32) for _ in range(2)])


def test_xcd_kernel_expert_weights_scale(orc):
    """expert_weights_scale = 2.5 (core/runtime.cpp:896-897): weights scaled
    after the normalisation."""
    note("XCD kernel: expert_weights_scale 2.5, 2 layers E=32, 2 tokens vs oracle")
    layers = [GpuLayer(H, 32, 8, F, (Q4_K,) * 3, seed=880 + i) for i in range(2)]
    for g in layers:
        g.layer.expert_weights_scale = 2.5
        g.host.scale = 2.5
    stack = make_stack(layers)
    rng = np.random.default_rng(14)
    for t in range(2):
        x = rng.standard_normal(H).astype(np.float32)
        out, xo, ids, w = stack(torch.from_numpy(x).to(DEV))
        torch.cuda.synchronize()
        xr = x.reshape(1, -1)
        for l, g in enumerate(layers):
            r = orc.moe_layer(g.host, xr, rms_eps=1e-6, scale=2.5)
            assert np.array_equal(ids[l].cpu().numpy(), r["ids"][0]), f"token {t} layer {l} ids"
            assert np.array_equal(bits(w[l].cpu().numpy()), bits(r["weights"][0])), f"token {t} layer {l} w"
            xr = r["xnext"]
        assert np.array_equal(bits(out.cpu().numpy()), bits(r["out"][0]))
    assert stack.status() & ~1 == 0
    stack.close()


def test_xcd_kernel_equals_other_kernels():
    """8 layers at the 30B shape, 4 tokens: the XCD kernel with XCD-local
    exchange words, with device-scope words, and the per-CU kernel give the
    same bits."""
    note("XCD kernel vs device-scope variant vs per-CU kernel: 8 layers 30B shape, 4 tokens")
    layers = [GpuLayer(H, 128, 8, F, (Q4_K,) * 3, seed=900 + i) for i in range(8)]
    xs = torch.empty((4, H), dtype=torch.float32, device=DEV)
    ops.randn_(xs, 98, 0.0, 1.0)
    xs = [xs[t].contiguous() for t in range(4)]
    s2 = make_stack(layers)
    s3 = make_stack(layers, {"QWMOE_DECODE_XCD_LOCAL": "0"})
    s1 = make_stack(layers, {"QWMOE_DECODE_XCD": "0"})
    assert (s2.kernel(), s3.kernel(), s1.kernel()) == (2, 3, 1)
    r2, r3, r1 = run_tokens(s2, xs), run_tokens(s3, xs), run_tokens(s1, xs)
    same_bits(r2, r3)
    same_bits(r2, r1)
    for s in (s1, s2, s3):
        assert s.status() & ~1 == 0
        s.close()


def test_xcd_kernel_after_odd_sized_launches():
    """The dispatcher deals workgroups to the XCDs round robin from where the
    previous dispatch stopped, so one-workgroup launches before the stack shift
    which XCD workgroup 0 lands on.  Every shift: the same bits as the per-CU
    kernel and no status bit beyond the tie replay."""
    note("XCD kernel after 0..7 one-workgroup launches: 2 layers 30B shape vs per-CU kernel")
    layers = [GpuLayer(H, 128, 8, F, (Q4_K,) * 3, seed=920 + i) for i in range(2)]
    s2 = make_stack(layers)
    s1 = make_stack(layers, {"QWMOE_DECODE_XCD": "0"})
    assert (s2.kernel(), s1.kernel()) == (2, 1)
    x = torch.empty(H, dtype=torch.float32, device=DEV)
    ops.randn_(x, 77, 0.0, 1.0)
    ref = run_tokens(s1, [x])
    pad = torch.empty(255, dtype=torch.float32, device=DEV)   # one workgroup of k_randn
    for r in range(8):
        for i in range(r):
            ops.randn_(pad, 100 + i, 0.0, 1.0)
        same_bits(ref, run_tokens(s2, [x]))
        assert s2.status() & ~1 == 0, f"shift {r}: status {s2.status()}"
    s1.close()
    s2.close()
