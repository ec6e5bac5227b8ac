"""GPU parity of the attention half of Seg A (qwmoe_attn_seg) and of one whole
Qwen3-MoE decoder layer (qwmoe_decoder_layer), through the C ABI.

The bar (north_star: fp32 outputs within 1e-3 of the ggml CPU path):
attn_resid and ffn_in within 1e-3 of the reference's magnitude, against ggml's
own graph (oracle/_ref, when built) and against the CPU restatement
(oracle_lib.attn_seg_restated, pinned to ggml in test_attn_oracle.py); the f16
cache rows the call writes: V bit for bit, K within one f16 step.

* the 30B-A3B attention shape (H = 2048, 32 query / 4 kv heads, D = 128,
  Q4_K q/k/o, Q6_K v): decode at n_past 0, 37 and 700, a T = 5 verify batch,
  T = 64 and T = 37 prefill chunks (the matrix-core products), and decode at
  n_past 3000 (many P.V partial sums);
* the decoder layer equals its parts (attn_seg -> ffn_layer -> residual add)
  bit for bit, and the whole layer matches ggml's attention graph followed by
  ggml's MoE layer within 1e-3 where both route the same experts.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from questwend_amd import ops  # noqa: E402
from oracle_lib import (AttnWeights, Oracle, Q4_K, Q6_K, RefGGML, attn_seg_restated, have_ref)  # noqa: E402
from test_gpu_decode import GpuLayer, bits  # noqa: E402

DEV = "cuda:0"
H, NH, NKV, D = 2048, 32, 4, 128
TYPES = (Q4_K, Q4_K, Q6_K, Q4_K)
TOL = 1e-3


def note(msg: str) -> None:
    print(f"[gpu-attn] {msg}", flush=True)


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
def orc():
    return Oracle()


def rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


class GpuAttn:
    """AttnWeights on the device with f16 caches of n_ctx rows."""

    def __init__(self, aw: AttnWeights, n_ctx: int, kc0=None, vc0=None):
        self.aw, self.n_ctx = aw, n_ctx
        NK = aw.n_head_kv * aw.D
        self.kc_host = np.zeros((n_ctx, NK), np.uint16) if kc0 is None else kc0.copy()
        self.vc_host = np.zeros((n_ctx, NK), np.uint16) if vc0 is None else vc0.copy()
        self.t = [dev(x) for x in (aw.attn_norm, aw.wq, aw.wk, aw.wv, aw.wo, aw.q_norm, aw.k_norm, aw.ffn_norm)]
        self.kc = dev(self.kc_host.view(np.int16))
        self.vc = dev(self.vc_host.view(np.int16))
        an, wq, wk, wv, wo, qn, kn, fn = self.t
        self.layer = ops.make_attn_layer(aw.H, aw.n_head, aw.n_head_kv, aw.D, an, wq, wk, wv, wo, aw.types, qn, kn,
                                         fn, self.kc, self.vc, aw.freq_base)

    def caches(self):
        return self.kc.cpu().numpy().view(np.uint16), self.vc.cpu().numpy().view(np.uint16)


def reference(orc, aw, h, n_past, kc, vc):
    if have_ref():
        return RefGGML().attn_seg(aw, h, n_past, kc, vc, n_threads=16)
    return attn_seg_restated(aw, h, n_past, kc, vc, orc)


def check_step(orc, g: GpuAttn, h, n_past, what):
    T = h.shape[0]
    kc_ref, vc_ref = g.kc_host.copy(), g.vc_host.copy()
    r_res, r_fin, _, _ = reference(orc, g.aw, h, n_past, kc_ref, vc_ref)
    kc_o, vc_o = g.kc_host.copy(), g.vc_host.copy()
    o_res, o_fin, _, _ = attn_seg_restated(g.aw, h, n_past, kc_o, vc_o, orc)
    res, fin = ops.attn_seg(g.layer, dev(h), n_past)
    torch.cuda.synchronize()
    res, fin = res.cpu().numpy(), fin.cpu().numpy()
    kc, vc = g.caches()
    e = (rel(res, r_res), rel(fin, r_fin), rel(res, o_res), rel(fin, o_fin))
    note(f"  {what}: rel err vs reference resid {e[0]:.2e} ffn_in {e[1]:.2e}; vs restatement {e[2]:.2e} {e[3]:.2e}")
    assert max(e) < TOL, f"{what}: {e}"
    rows = slice(n_past, n_past + T)
    assert np.array_equal(vc[rows], vc_ref[rows]), f"{what}: V cache rows"
    dk = np.abs(kc[rows].view(np.float16).astype(np.float64) - kc_ref[rows].view(np.float16).astype(np.float64))
    assert np.all(dk <= np.spacing(np.abs(kc_ref[rows].view(np.float16))).astype(np.float64)), f"{what}: K cache rows"
    assert np.array_equal(kc[:n_past], g.kc_host[:n_past]) and np.array_equal(vc[:n_past], g.vc_host[:n_past])
    # carry the reference's caches forward (the next step reads them)
    g.kc_host[rows], g.vc_host[rows] = kc_ref[rows], vc_ref[rows]
    g.kc.copy_(dev(g.kc_host.view(np.int16)))
    g.vc.copy_(dev(g.vc_host.view(np.int16)))
    return res, fin


def filled_caches(n_ctx, n_fill, seed):
    rng = np.random.default_rng(seed)
    kc = np.zeros((n_ctx, NKV * D), np.uint16)
    vc = np.zeros((n_ctx, NKV * D), np.uint16)
    kc[:n_fill] = (rng.standard_normal((n_fill, NKV * D)) * 0.5).astype(np.float16).view(np.uint16)
    vc[:n_fill] = (rng.standard_normal((n_fill, NKV * D)) * 0.5).astype(np.float16).view(np.uint16)
    return kc, vc


def test_attn_seg_30b_shape_steps(orc):
    note(f"attn_seg 30B shape (H={H}, {NH}/{NKV} heads, D={D}, Q4_K/Q6_K): decode, verify, prefill chunk")
    aw = AttnWeights(H, NH, NKV, D, TYPES, seed=3, oracle=orc)
    kc, vc = filled_caches(1024, 700, seed=9)
    g = GpuAttn(aw, 1024, kc, vc)
    rng = np.random.default_rng(1)
    # T = 64 and 37 take the matrix-core products (at least 64 query rows), 37 with
    # a ragged last row block; the others the decode kernels
    for T, n_past in ((1, 0), (1, 37), (5, 40), (64, 100), (37, 164), (1, 700)):
        check_step(orc, g, rng.standard_normal((T, H)).astype(np.float32), n_past, f"T={T} n_past={n_past}")


def test_attn_seg_long_context(orc):
    note("attn_seg 30B shape, decode at n_past=3000 (P.V in 47 partial sums)")
    aw = AttnWeights(H, NH, NKV, D, TYPES, seed=4, oracle=orc)
    kc, vc = filled_caches(4096, 3000, seed=10)
    g = GpuAttn(aw, 4096, kc, vc)
    check_step(orc, g, np.random.default_rng(2).standard_normal((1, H)).astype(np.float32), 3000, "T=1 n_past=3000")


def test_attn_seg_small_heads(orc):
    note("attn_seg H=512, 8/2 heads, T=3 at n_past=5, Q8_0 q/k/v/o")
    from oracle_lib import Q8_0
    aw = AttnWeights(512, 8, 2, D, (Q8_0,) * 4, seed=6, oracle=orc)
    kc = np.zeros((64, 2 * D), np.uint16)
    vc = np.zeros((64, 2 * D), np.uint16)
    rng = np.random.default_rng(3)
    kc[:5] = (rng.standard_normal((5, 2 * D)) * 0.5).astype(np.float16).view(np.uint16)
    vc[:5] = (rng.standard_normal((5, 2 * D)) * 0.5).astype(np.float16).view(np.uint16)
    g = GpuAttn(aw, 64, kc, vc)
    check_step(orc, g, rng.standard_normal((3, 512)).astype(np.float32), 5, "T=3 n_past=5")


@pytest.mark.parametrize("T", [1, 5])
def test_decoder_layer(orc, T):
    note(f"decoder layer (attention + MoE FFN + residual), 30B shape, T={T}")
    aw = AttnWeights(H, NH, NKV, D, TYPES, seed=20 + T, oracle=orc)
    kc, vc = filled_caches(256, 50, seed=T)
    g = GpuAttn(aw, 256, kc, vc)
    moe = GpuLayer(H, 128, 8, 768, (Q4_K,) * 3, seed=60 + T)
    h = np.random.default_rng(T).standard_normal((T, H)).astype(np.float32)
    # the layer, then its parts on a second copy of the caches: the same bits
    out, ids, w = ops.decoder_layer(g.layer, moe.layer, dev(h), 50)
    torch.cuda.synchronize()
    g2 = GpuAttn(aw, 256, kc, vc)
    res, fin = ops.attn_seg(g2.layer, dev(h), 50)
    mo, _, ids2, w2 = ops.ffn_layer(moe.layer, fin)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2) and torch.equal(w.view(torch.int32), w2.view(torch.int32))
    assert torch.equal(out.view(torch.int32), (mo + res).view(torch.int32))
    assert torch.equal(g.kc, g2.kc) and torch.equal(g.vc, g2.vc)
    # against the reference: ggml's attention graph, then the MoE layer on its ffn_in
    r_res, r_fin, _, _ = reference(orc, aw, h, 50, kc.copy(), vc.copy())
    r = orc.moe_layer(moe.host, r_fin, rms_eps=-1.0)
    want = r["out"] + r_res
    same = np.all(ids.cpu().numpy() == r["ids"], axis=1)
    note(f"  tokens routed alike: {int(same.sum())}/{T}")
    assert same.sum() >= max(1, T - 1)
    e = rel(out.cpu().numpy()[same], want[same])
    note(f"  layer output rel err vs reference {e:.2e}")
    assert e < TOL
