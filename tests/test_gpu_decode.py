"""GPU parity of the persistent whole-stack decode kernel (qwmoe_decode_stack_*).

Free-running: each layer consumes the previous layer's normalized output, with
no teacher forcing; every layer's router ids and weights, the last layer's
output and its RMSNorm must equal the CPU oracle bit for bit.  Weights are
produced by the GPU quantizer (itself checked byte for byte against the oracle
in test_gpu_parity.py) and copied to the host for the oracle.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from questwend_amd import ops  # noqa: E402
from oracle_lib import Q4_K, Q6_K, LayerWeights, Oracle, row_size  # noqa: E402

DEV = "cuda:0"


def note(msg: str) -> None:
    print(f"[gpu-decode] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    prev = ops.set_mfma_form(ops.MFMA_EXACT)   # bit-exact tests: heavy bins on the matrix cores replay ggml's float steps
    yield
    torch.cuda.synchronize()
    ops.set_mfma_form(prev)


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


class GpuLayer:
    """One layer's synthetic weights generated and quantized on the GPU, plus a
    host copy of the same bytes in the oracle's LayerWeights form."""

    def __init__(self, H, E, k, F, types, seed, permute=False, dup_router=False):
        tg, tu, td = types
        self.router = torch.empty((E, H), dtype=torch.float32, device=DEV)
        ops.randn_(self.router, seed * 10 + 1, 0.0, 0.02)
        if dup_router:   # experts 2j and 2j+1 get equal logits: every top-k has ties
            self.router[1::2] = self.router[0::2]
        mats = []
        tmp = torch.empty(E * F * H, dtype=torch.float32, device=DEV)
        for j, (t, rows, cols) in enumerate(((tg, F, H), (tu, F, H), (td, H, F))):
            ops.randn_(tmp, seed * 10 + 2 + j, 0.0, 0.02)
            mats.append(ops.quantize_chunk(t, tmp.view(E * rows, cols)).view(E, -1))
        del tmp
        self.slots = None
        if permute:
            g = torch.Generator().manual_seed(seed)
            perms = [torch.randperm(E, generator=g).to(torch.int32) for _ in range(3)]
            pools = []
            for m, p in zip(mats, perms):
                pool = torch.empty_like(m)
                pool[p.long().to(DEV)] = m       # logical expert e lives in slot p[e]
                pools.append(pool)
            self.slots = tuple(p.to(DEV) for p in perms)
            mats_dev = pools
        else:
            mats_dev = mats
        self.gate, self.up, self.down = mats_dev
        self.layer = ops.make_layer(H, E, k, F, self.router, self.gate, self.up, self.down, types,
                                    n_slots=(E, E, E), slots=self.slots)
        torch.cuda.synchronize()
        lw = LayerWeights.__new__(LayerWeights)
        lw.H, lw.E, lw.k, lw.F = H, E, k, F
        lw.type_gate, lw.type_up, lw.type_down = types
        lw.router = self.router.cpu().numpy()
        lw.gate, lw.up, lw.down = (m.cpu().numpy().reshape(-1) for m in mats_dev)
        lw.n_slots = E
        lw.slot_of = None if self.slots is None else tuple(s.cpu().numpy() for s in self.slots)
        self.host = lw


def run_and_compare(orc, layers, tokens, eps=1e-6):
    stack = ops.DecodeStack([g.layer for g in layers], eps, keepalive=layers)
    for t, x in enumerate(tokens):
        out, xo, ids, w = stack(torch.from_numpy(x).to(DEV))
        torch.cuda.synchronize()
        xr = x.reshape(1, -1)
        ids_h, w_h = ids.cpu().numpy(), w.cpu().numpy()
        for l, g in enumerate(layers):
            r = orc.moe_layer(g.host, xr, rms_eps=eps)
            assert np.array_equal(ids_h[l], r["ids"][0]), f"token {t} layer {l} ids"
            assert np.array_equal(bits(w_h[l]), bits(r["weights"][0])), f"token {t} layer {l} weights"
            xr = r["xnext"]
        assert np.array_equal(bits(out.cpu().numpy()), bits(r["out"][0])), f"token {t} out"
        assert np.array_equal(bits(xo.cpu().numpy()), bits(r["xnext"][0])), f"token {t} x_out"
    st = stack.status()
    assert st & ~1 == 0, f"decode stack status {st}"
    stack.close()


def test_decode_stack_small(orc):
    note("decode stack: 3 layers H=1024 E=16 k=4 F=512 Q4_K, 3 tokens")
    layers = [GpuLayer(1024, 16, 4, 512, (Q4_K,) * 3, seed=300 + i) for i in range(3)]
    rng = np.random.default_rng(0)
    run_and_compare(orc, layers, [rng.standard_normal(1024).astype(np.float32) for _ in range(3)])


def test_decode_stack_30b_shape(orc):
    note("decode stack: 2 layers of the 30B-A3B shape (H=2048 E=128 k=8 F=768 Q4_K), 2 tokens")
    layers = [GpuLayer(2048, 128, 8, 768, (Q4_K,) * 3, seed=400 + i) for i in range(2)]
    rng = np.random.default_rng(1)
    run_and_compare(orc, layers, [rng.standard_normal(2048).astype(np.float32) for _ in range(2)])


def test_decode_stack_q6k_down_permuted_slots(orc):
    note("decode stack: Q6_K down, permuted slot pools, 2 layers H=1024 E=16 k=8 F=512")
    layers = [GpuLayer(1024, 16, 8, 512, (Q4_K, Q4_K, Q6_K), seed=500 + i, permute=True) for i in range(2)]
    rng = np.random.default_rng(2)
    run_and_compare(orc, layers, [rng.standard_normal(1024).astype(np.float32) for _ in range(2)])


def test_decode_stack_router_ties(orc):
    """Router rows equal in pairs: every layer's probabilities tie in pairs, inside
    the first k places and (k odd) across the k-th place, so the kernel's
    speculative order (by logit, ties by index) fails its check and the exact
    order comes from the std::sort replay; where that order differs from the
    speculative one the gate/up rows are loaded again."""
    note("decode stack: tied router logits, 3 layers H=1024 E=16 k=3 F=512, 3 tokens")
    layers = [GpuLayer(1024, 16, 3, 512, (Q4_K,) * 3, seed=700 + i, dup_router=True) for i in range(3)]
    rng = np.random.default_rng(3)
    run_and_compare(orc, layers, [rng.standard_normal(1024).astype(np.float32) for _ in range(3)])


def test_decode_stack_equals_per_layer_path():
    """8 layers at the 30B shape: the persistent kernel and the per-layer
    qwmoe_ffn_layer path agree bit for bit over 4 tokens."""
    note("decode stack vs per-layer path: 8 layers 30B shape, 4 tokens")
    layers = [GpuLayer(2048, 128, 8, 768, (Q4_K,) * 3, seed=600 + i) for i in range(8)]
    stack = ops.DecodeStack([g.layer for g in layers], 1e-6, keepalive=layers)
    xs = torch.empty((4, 2048), dtype=torch.float32, device=DEV)
    ops.randn_(xs, 99, 0.0, 1.0)
    for t in range(4):
        out, xo, ids, w = stack(xs[t].contiguous())
        x = xs[t:t + 1].contiguous()
        for l, g in enumerate(layers):
            o, xn, i2, w2 = ops.ffn_layer(g.layer, x, rms_eps=1e-6)
            torch.cuda.synchronize()
            assert torch.equal(ids[l], i2[0]), f"token {t} layer {l}"
            assert torch.equal(w[l].view(torch.int32), w2[0].view(torch.int32))
            x = xn
        assert torch.equal(out.view(torch.int32), o[0].view(torch.int32))
        assert torch.equal(xo.view(torch.int32), x[0].view(torch.int32))
    assert stack.status() & ~1 == 0
    stack.close()


def test_decode_stack_rejects_unsupported_shapes():
    note("decode stack argument checks")
    g = GpuLayer(512, 12, 2, 256, (Q4_K,) * 3, seed=7)      # E % 8 != 0
    with pytest.raises(qa.QwmoeError):
        ops.DecodeStack([g.layer], 1e-6)
