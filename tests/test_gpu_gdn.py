"""GPU parity of the gated-delta-net half of Seg A (qwmoe_gdn_seg, the
recurrent layers of qwen3next / qwen35moe) through the C ABI.

The bar (north_star: fp32 outputs within 1e-3 of the ggml CPU path):
attn_resid and ffn_in within 1e-3 of the reference's magnitude, and both states
the call leaves (conv state, recurrent state) within 1e-3, against ggml's own
graph for the block (oracle/_ref's qwref_gdn_seg, when built) and against the
CPU restatement (oracle_lib.gdn_seg_restated, pinned to ggml in
test_gdn_oracle.py).  The conv state is a copy of projection outputs (the
quantized row dots, ggml's bits), so it is checked bit for bit.

* the shape in the reference's build_gdn comments (H = 2048, S = 128, 16 key and
  16 value heads, d_conv = 4: conv_ch 6144) with Q4_K / Q6_K / Q8_0 projections:
  decode from a zero and from a random state, a T = 5 batch, T = 64 and T = 300
  chunks (the matrix-core projections);
* 32 value heads over 16 key heads (value head h reads key head h % 16, as
  ggml's op broadcasts), decode and T = 17;
* calls chain through the states: T = 3, 1, 4 equal one T = 8 call within the bar.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from questwend_amd import ops  # noqa: E402
from oracle_lib import GdnWeights, Oracle, Q4_K, Q6_K, Q8_0, RefGGML, gdn_seg_restated, have_ref  # noqa: E402

DEV = "cuda:0"
TOL = 1e-3


def note(msg: str) -> None:
    print(f"[gpu-gdn] {msg}", flush=True)


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
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(float(np.max(np.abs(b))), 1e-30))


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


class GpuGdn:
    """GdnWeights on the device with their two states."""

    def __init__(self, gw: GdnWeights, conv_state, ssm_state):
        self.gw = gw
        self.t = [dev(x) for x in (gw.attn_norm, gw.w_qkv, gw.w_gate, gw.w_beta, gw.w_alpha, gw.w_out, gw.dt_bias,
                                   gw.ssm_a, gw.conv1d, gw.ssm_norm, gw.ffn_norm)]
        self.cs = dev(conv_state)
        self.ss = dev(ssm_state)
        an, wq, wg, wb, wa, wo, dtb, sa, c1, sn, fn = self.t
        self.layer = ops.make_gdn_layer(gw.H, gw.S, gw.H_k, gw.H_v, gw.d_conv, gw.types, an, wq, wg, wb, wa, wo,
                                        dtb, sa, c1, sn, fn, self.cs, self.ss)

    def run(self, h):
        resid, fin = ops.gdn_seg(self.layer, dev(h))
        torch.cuda.synchronize()
        return resid.cpu().numpy(), fin.cpu().numpy()

    def states(self):
        return self.cs.cpu().numpy(), self.ss.cpu().numpy()


SHAPE16 = dict(H=2048, S=128, H_k=16, H_v=16, d_conv=4)
TYPES = (Q4_K, Q6_K, Q8_0, Q8_0, Q4_K)


def check(gw, orc, h, rand_state: bool, label: str):
    cs0, ss0 = gw.fresh_state(np.random.default_rng(5) if rand_state else None)
    g = GpuGdn(gw, cs0, ss0)
    got = g.run(h)
    gcs, gss = g.states()
    cs_r, ss_r = cs0.copy(), ss0.copy()
    want_r = gdn_seg_restated(gw, h, cs_r, ss_r, orc)
    e_r = (rel(got[0], want_r[0]), rel(got[1], want_r[1]), rel(gss, ss_r))
    msg = f"{label}: vs restatement resid {e_r[0]:.2e} ffn_in {e_r[1]:.2e} state {e_r[2]:.2e}"
    assert np.array_equal(gcs, cs_r), label
    if have_ref():
        cs_g, ss_g = cs0.copy(), ss0.copy()
        want_g = RefGGML().gdn_seg(gw, h, cs_g, ss_g)
        e_g = (rel(got[0], want_g[0]), rel(got[1], want_g[1]), rel(gss, ss_g))
        msg += f"; vs reference resid {e_g[0]:.2e} ffn_in {e_g[1]:.2e} state {e_g[2]:.2e}"
        assert np.array_equal(gcs, cs_g), label
        assert max(e_g) < TOL, msg
    note(msg)
    assert max(e_r) < TOL, msg
    assert ops.device_status(clear=True) == 0


@pytest.mark.parametrize("T,rand_state", [(1, False), (1, True), (5, True), (64, True), (300, True)])
def test_gdn_seg_16_heads(orc, T, rand_state):
    gw = GdnWeights(**SHAPE16, types=TYPES, seed=21, oracle=orc)
    h = np.random.default_rng(100 + T).standard_normal((T, gw.H)).astype(np.float32)
    check(gw, orc, h, rand_state, f"H_v=16 T={T} random state={rand_state}")


@pytest.mark.parametrize("T", [1, 17])
def test_gdn_seg_value_heads_broadcast(orc, T):
    gw = GdnWeights(2048, 128, 16, 32, 4, (Q4_K, Q4_K, Q8_0, Q8_0, Q6_K), 31, orc)
    h = np.random.default_rng(200 + T).standard_normal((T, gw.H)).astype(np.float32)
    check(gw, orc, h, True, f"H_v=32 over H_k=16 T={T}")


def test_gdn_calls_chain_through_the_states(orc):
    gw = GdnWeights(**SHAPE16, types=TYPES, seed=41, oracle=orc)
    h = np.random.default_rng(7).standard_normal((8, gw.H)).astype(np.float32)
    cs0, ss0 = gw.fresh_state(np.random.default_rng(8))
    whole = GpuGdn(gw, cs0, ss0)
    w_out = whole.run(h)
    parts = GpuGdn(gw, cs0, ss0)
    p_out = [parts.run(h[a:b]) for a, b in ((0, 3), (3, 4), (4, 8))]
    resid = np.concatenate([p[0] for p in p_out])
    e = rel(resid, w_out[0])
    e_s = rel(parts.states()[1], whole.states()[1])
    note(f"T = 3, 1, 4 against T = 8: resid {e:.2e}, state {e_s:.2e}")
    assert e < TOL and e_s < TOL
    assert np.array_equal(parts.states()[0], whole.states()[0])
