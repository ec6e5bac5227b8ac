"""Persistent launches and HIP graph capture (qwmoe_decode_stack_run,
qwmoe_layer_stack_run).

Each persistent launch takes a fresh exchange epoch from the host, so a launch
recorded into a graph would replay the same epoch and accept the words its
previous replay left.  On a capturing stream the decode stack therefore
refuses the call (QWMOE_ERR_UNSUPPORTED, nothing enqueued) and the layer stack
records its per-layer chain instead of the persistent kernels.  Checked here:

* decode stack: the status under capture, and a graph recorded around the
  refused call replays without touching the stack;
* layer stack (two 30B-A3B Q4_K layers, where T = 1 and T = 4 run on the
  persistent decode and verify kernels outside capture): graphs captured at
  T = 1 and T = 4, each replayed four times with new inputs, with eager library
  work and synchronisations between the replays, equal the eager runs (which
  take the persistent kernels) bit for bit on every replay.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from questwend_amd import lib, ops  # noqa: E402
from oracle_lib import Q4_K  # noqa: E402
from test_gpu_decode import GpuLayer  # noqa: E402

DEV = "cuda:0"


def note(msg: str) -> None:
    print(f"[gpu-capture] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    prev = ops.set_mfma_form(ops.MFMA_EXACT)
    yield
    torch.cuda.synchronize()
    ops.set_mfma_form(prev)


@pytest.fixture(scope="module")
def layers30b():
    return [GpuLayer(2048, 128, 8, 768, (Q4_K,) * 3, seed=1200 + i) for i in range(2)]


def test_decode_stack_refuses_capture(layers30b):
    note("decode stack under capture: QWMOE_ERR_UNSUPPORTED, nothing enqueued")
    Ls = [g.layer for g in layers30b]
    dstack = ops.DecodeStack(Ls, 1e-6, keepalive=layers30b)
    x = torch.randn(2048, device=DEV)
    out = torch.zeros(2048, device=DEV)
    ref, _, _, _ = dstack(x)
    torch.cuda.synchronize()
    y = torch.zeros(4, device=DEV)
    g = torch.cuda.CUDAGraph()
    rc = None
    with torch.cuda.graph(g):
        y.add_(1.0)
        rc = lib().qwmoe_decode_stack_run(ops.stream(), dstack.h, C.c_void_p(x.data_ptr()),
                                          C.c_void_p(out.data_ptr()), None, None, None)
    assert rc == -2, f"decode stack run under capture returned {rc}"
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, torch.full((4,), 3.0, device=DEV))   # the graph ran: three replays, capture runs nothing
    assert torch.equal(out, torch.zeros(2048, device=DEV))     # the stack's kernel was never recorded
    again, _, _, _ = dstack(x)
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int32), ref.view(torch.int32))
    assert dstack.status() & ~1 == 0
    dstack.close()


@pytest.mark.parametrize("T", [1, 4])
def test_layer_stack_capture_replays_equal_eager(layers30b, T):
    note(f"layer stack: a graph captured at T={T} (per-layer chain) vs eager persistent runs, 4 replays")
    Ls = [g.layer for g in layers30b]
    stack = ops.LayerStack(Ls, 1e-6, max_tokens=5, keepalive=layers30b)
    rng = np.random.default_rng(30 + T)
    xs = torch.zeros((T, 2048), device=DEV)
    # warm-up outside capture (creates the T = 1 decode stack lazily)
    stack(xs.copy_(torch.from_numpy(rng.standard_normal((T, 2048)).astype(np.float32))))
    torch.cuda.synchronize()
    if T == 1:
        assert stack.kernel_t1() in (2, 3), "T = 1 should run on the XCD decode kernel outside capture"
    else:
        assert stack.kernel() in (2, 3), "T = 4 should run on the persistent verify kernel outside capture"
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        go, gxo, gids, gw = stack(xs)
    for i in range(4):
        x = torch.from_numpy(rng.standard_normal((T, 2048)).astype(np.float32)).to(DEV)
        xs.copy_(x)
        g.replay()
        if i % 2 == 0:
            torch.cuda.synchronize()
        # eager library work between replays, on the same stream and workspace
        ops.ffn_layer(Ls[i % 2], torch.from_numpy(rng.standard_normal((3, 2048)).astype(np.float32)).to(DEV),
                      rms_eps=1e-6)
        eo, exo, eids, ew = stack(x)
        torch.cuda.synchronize()
        assert torch.equal(gids, eids), f"replay {i}: ids"
        assert torch.equal(gw.view(torch.int32), ew.view(torch.int32)), f"replay {i}: weights"
        assert torch.equal(go.view(torch.int32), eo.view(torch.int32)), f"replay {i}: out"
        assert torch.equal(gxo.view(torch.int32), exo.view(torch.int32)), f"replay {i}: x_out"
    assert stack.status() & ~1 == 0
    stack.close()
