"""GPU parity of resident-only routing (core/runtime.cpp:870-881, the
cache_fast_build && resident_decode branch of build_moe): the router records
want = argsort_top_k of the raw logits, then adds the layer's mask row (0 for
a resident expert, -inf for an absent one) before the softmax, so top-k never
picks an absent expert.  Through the C ABI: qwmoe_router_topk_resident, and the
qwmoe_layer fields resmask / want_ids of qwmoe_ffn_layer, the layer stack and
the persistent decode stacks.  Bit for bit against the CPU oracle, whose
resident router tests/test_oracle.py pins to ggml's graph of the same ops.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from questwend_amd import ops  # noqa: E402
from oracle_lib import Q4_K, Q6_K, LayerWeights, Oracle  # noqa: E402

DEV = "cuda:0"


def note(msg: str) -> None:
    print(f"[gpu-resident] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    prev = ops.set_mfma_form(ops.MFMA_EXACT)   # bit-exact layer outputs when bins reach the matrix cores
    yield
    torch.cuda.synchronize()
    ops.set_mfma_form(prev)


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.int32)


def resident_mask(rng, E: int, n_res: int) -> tuple[np.ndarray, np.ndarray]:
    res = np.sort(rng.choice(E, n_res, replace=False))
    mask = np.full(E, -np.inf, np.float32)
    mask[res] = 0.0
    return mask, res


@pytest.mark.parametrize("E,k,T,n_res", [(128, 8, 1, 40), (128, 8, 3, 8), (128, 8, 20, 100), (64, 4, 40, 64),
                                         (256, 8, 2, 9)])
def test_router_resident(orc, E, k, T, n_res):
    """T <= 16 and E <= 128 take the fused top-k + grouping launch inside the
    layer; the router entry point runs the per-token top-k kernel."""
    note(f"resident router E={E} k={k} T={T} resident={n_res}")
    rng = np.random.default_rng(E + k + T + n_res)
    H = 512
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    mask, res = resident_mask(rng, E, n_res)
    ids, w, want = ops.router_topk_resident(dev(W), dev(x), k, dev(mask))
    i2, w2, want2, _ = orc.router_resident(W, x, k, mask)
    assert np.array_equal(host(want), want2)
    assert np.array_equal(host(ids), i2)
    assert np.array_equal(bits(host(w)), bits(w2))
    assert np.isin(host(ids), res).all()
    # no mask: want equals the selection
    ids0, w0, want0 = ops.router_topk_resident(dev(W), dev(x), k, None)
    assert np.array_equal(host(want0), host(ids0))
    i3, w3, _, _ = orc.router(W, x, k)
    assert np.array_equal(host(ids0), i3) and np.array_equal(bits(host(w0)), bits(w3))


def gpu_layer(lw: LayerWeights, resmask=None, want=None):
    tensors = [dev(lw.router), dev(lw.gate), dev(lw.up), dev(lw.down)]
    slots = None if lw.slot_of is None else tuple(dev(s) for s in lw.slot_of)
    L = ops.make_layer(lw.H, lw.E, lw.k, lw.F, *tensors, (lw.type_gate, lw.type_up, lw.type_down),
                       n_slots=(lw.n_slots,) * 3, slots=slots, resmask=resmask, want_ids=want)
    return L, tensors + ([] if slots is None else list(slots))


@pytest.mark.parametrize("T,n_res,types", [(1, 24, (Q4_K, Q4_K, Q4_K)), (5, 12, (Q4_K, Q4_K, Q6_K)),
                                           (33, 30, (Q4_K, Q4_K, Q4_K))])
def test_ffn_layer_resident(orc, T, n_res, types):
    """qwmoe_ffn_layer with resmask / want_ids: ids, weights, want and the layer
    output bit-identical to the oracle's layer with the same mask (T = 33 puts
    bins on the matrix cores, exact form)."""
    note(f"ffn_layer resident T={T} resident={n_res} types={types}")
    E, k = 32, 8
    lw = LayerWeights(1024, E, k, 512, *types, seed=500 + T, oracle=orc, permute=True)
    rng = np.random.default_rng(T)
    mask, res = resident_mask(rng, E, n_res)
    md = dev(mask)
    want = torch.full((T, k), -1, dtype=torch.int32, device=DEV)
    L, keep = gpu_layer(lw, md, want)
    x = rng.standard_normal((T, lw.H)).astype(np.float32)
    prev = ops.set_mfma_min_rows(8)
    try:
        out, xn, ids, w = ops.ffn_layer(L, dev(x), rms_eps=1e-6)
    finally:
        ops.set_mfma_min_rows(prev)
    r = orc.moe_layer(lw, x, rms_eps=1e-6, resmask=mask)
    assert np.array_equal(host(want), r["want"])
    assert np.array_equal(host(ids), r["ids"])
    assert np.isin(host(ids), res).all()
    assert np.array_equal(bits(host(w)), bits(r["weights"]))
    assert np.array_equal(bits(host(out)), bits(r["out"]))
    assert ops.device_status(clear=True) & (qa.STATUS_BAD_ID | qa.STATUS_BAD_SLOT) == 0


def masked_layers(layers, n_res_list, seed, T=1):
    """ctypes copies of GpuLayer descriptors with a resident mask row and a want
    buffer each; returns (descriptors, masks (host), wants (device), keepalive)."""
    rng = np.random.default_rng(seed)
    descs, masks, wants, keep = [], [], [], []
    for g, n_res in zip(layers, n_res_list):
        E, k = g.layer.n_expert, g.layer.n_expert_used
        mask, _ = resident_mask(rng, E, n_res)
        md = dev(mask)
        want = torch.full((T, k), -1, dtype=torch.int32, device=DEV)
        L = qa.Layer.from_buffer_copy(g.layer)
        L.resmask, L.want_ids = md.data_ptr(), want.data_ptr()
        descs.append(L)
        masks.append(mask)
        wants.append(want)
        keep += [md, want, g]
    return descs, masks, wants, keep


def chain_oracle(orc, layers, masks, x, eps=1e-6):
    """The stack on the CPU: each layer's oracle (with its mask) on the previous
    layer's RMSNorm output."""
    rs, xr = [], x
    for g, m in zip(layers, masks):
        r = orc.moe_layer(g.host, xr, rms_eps=eps, resmask=m)
        rs.append(r)
        xr = r["xnext"]
    return rs


@pytest.mark.parametrize("kernel_env", ["xcd", "per_cu"])
def test_decode_stack_resident(orc, kernel_env):
    """The persistent decode stack with every layer's mask and want: per layer
    ids / weights / want and the last layer's output bit-identical to the
    oracle chain; masks from 9 resident experts (ranks past k tie at -inf) to all
    128.  XCD kernel on a 256-CU device, else the per-CU kernel."""
    import os
    from test_gpu_decode import GpuLayer
    if kernel_env == "xcd" and torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the XCD kernel needs a 256-CU device")
    note(f"decode stack resident ({kernel_env}): 3 layers H=2048 E=128 k=8 F=768, 3 tokens")
    layers = [GpuLayer(2048, 128, 8, 768, (Q4_K,) * 3, seed=700 + i, permute=(i == 1)) for i in range(3)]
    descs, masks, wants, keep = masked_layers(layers, [9, 40, 128], seed=7)
    old = os.environ.get("QWMOE_DECODE_XCD")
    os.environ["QWMOE_DECODE_XCD"] = "1" if kernel_env == "xcd" else "0"
    try:
        stack = ops.DecodeStack(descs, 1e-6, keepalive=keep)
    finally:
        if old is None:
            os.environ.pop("QWMOE_DECODE_XCD")
        else:
            os.environ["QWMOE_DECODE_XCD"] = old
    assert stack.kernel() in ((1,) if kernel_env == "per_cu" else (2, 3))
    rng = np.random.default_rng(3)
    for t in range(3):
        x = rng.standard_normal(2048).astype(np.float32)
        out, xo, ids, w = stack(dev(x))
        rs = chain_oracle(orc, layers, masks, x.reshape(1, -1))
        ids_h, w_h = host(ids), host(w)
        for l, r in enumerate(rs):
            assert np.array_equal(host(wants[l])[0], r["want"][0]), f"token {t} layer {l} want"
            assert np.array_equal(ids_h[l], r["ids"][0]), f"token {t} layer {l} ids"
            assert np.array_equal(bits(w_h[l]), bits(r["weights"][0])), f"token {t} layer {l} weights"
        assert np.array_equal(bits(host(out)), bits(rs[-1]["out"][0])), f"token {t} out"
        assert np.array_equal(bits(host(xo)), bits(rs[-1]["xnext"][0])), f"token {t} x_out"
    assert stack.status() & ~1 == 0
    stack.close()


@pytest.mark.parametrize("T", [1, 3])
def test_layer_stack_resident(orc, T):
    """qwmoe_layer_stack (captured graph) with masks and wants: per layer ids,
    want and the last layer's output bit-identical to the oracle chain; a mask
    changed in place between runs is read by the replayed graph."""
    from test_gpu_decode import GpuLayer
    note(f"layer stack resident T={T}: 2 layers H=1024 E=32 k=4 F=512")
    layers = [GpuLayer(1024, 32, 4, 512, (Q4_K,) * 3, seed=800 + i) for i in range(2)]
    descs, masks, wants, keep = masked_layers(layers, [6, 20], seed=8, T=T)
    stack = ops.LayerStack(descs, 1e-6, max_tokens=T, keepalive=keep)
    rng = np.random.default_rng(T)
    for rep in range(2):
        if rep == 1:   # new palette: the mask tensors are updated in place
            for m, d in zip(masks, keep[0::3]):
                m[:] = resident_mask(rng, m.size, 10)[0]
                d.copy_(torch.from_numpy(m))
        x = rng.standard_normal((T, 1024)).astype(np.float32)
        out, xo, ids, w = stack(dev(x))
        rs = chain_oracle(orc, layers, masks, x)
        for l, r in enumerate(rs):
            assert np.array_equal(host(wants[l]), r["want"]), f"rep {rep} layer {l} want"
            assert np.array_equal(host(ids)[l], r["ids"]), f"rep {rep} layer {l} ids"
        assert np.array_equal(bits(host(out)), bits(rs[-1]["out"])), f"rep {rep} out"
    stack.close()
