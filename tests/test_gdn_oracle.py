"""CPU tests of the gated-delta-net restatement (oracle_lib.gdn_seg_restated)
against the reference's own ggml graph for it (qwref_gdn_seg in
oracle/ref_driver.cpp: build_segA + build_gdn, core/runtime.cpp:1976-1995 and
737-859, on ggml's CPU backend built from /root/reference).  The restatement
is the GPU tests' second checker; here it is pinned to ggml."""
from __future__ import annotations

import numpy as np
import pytest

from oracle_lib import Q4_K, Q6_K, Q8_0, GdnWeights, Oracle, RefGGML, gdn_seg_restated, have_ref

pytestmark = pytest.mark.skipif(not have_ref(), reason="oracle/_ref (the reference ggml) not built")


def rel(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(float(np.max(np.abs(a))), 1e-30))


@pytest.fixture(scope="module")
def orc():
    return Oracle()


@pytest.fixture(scope="module")
def ref():
    return RefGGML()


CASES = [
    # H, S, H_k, H_v, d_conv, types (qkv, gate, beta, alpha, out), T, random initial state
    (256, 64, 2, 4, 4, (Q8_0,) * 5, 1, False),
    (256, 64, 2, 4, 4, (Q4_K, Q4_K, Q8_0, Q8_0, Q4_K), 5, True),
    (512, 128, 2, 2, 4, (Q4_K, Q6_K, Q8_0, Q8_0, Q6_K), 17, True),
    (256, 128, 1, 2, 3, (Q8_0, Q8_0, Q8_0, Q8_0, Q8_0), 2, True),
]


@pytest.mark.parametrize("H,S,Hk,Hv,dc,types,T,rand", CASES)
def test_restatement_matches_ggml(orc, ref, H, S, Hk, Hv, dc, types, T, rand):
    """Outputs, the gated norm's output and both states after the call agree
    with ggml's graph to float rounding (the recurrence runs in float64 here,
    float32 in ggml); the conv state (a copy) bit for bit."""
    gw = GdnWeights(H, S, Hk, Hv, dc, types, 7 + T, orc)
    h = np.random.default_rng(T).standard_normal((T, H)).astype(np.float32)
    cs1, ss1 = gw.fresh_state(np.random.default_rng(2) if rand else None)
    cs2, ss2 = cs1.copy(), ss1.copy()
    r1 = ref.gdn_seg(gw, h, cs1, ss1)
    r2 = gdn_seg_restated(gw, h, cs2, ss2, orc)
    assert rel(r1[0], r2[0]) < 1e-5 and rel(r1[1], r2[1]) < 1e-5 and rel(r1[2], r2[2]) < 1e-5
    assert np.array_equal(cs1, cs2)
    assert rel(ss1, ss2) < 1e-5


def test_chunks_chain_through_the_states(orc, ref):
    """Five tokens in one call equal three then two with the states carried
    (ggml bit for bit: every step is per token or per state element)."""
    gw = GdnWeights(256, 64, 2, 4, 4, (Q8_0,) * 5, 11, orc)
    h = np.random.default_rng(3).standard_normal((5, 256)).astype(np.float32)
    cs, ss = gw.fresh_state(np.random.default_rng(4))
    a = ref.gdn_seg(gw, h, cs.copy(), ss_a := ss.copy())
    c2, s2 = cs.copy(), ss.copy()
    b1 = ref.gdn_seg(gw, h[:3], c2, s2)
    b2 = ref.gdn_seg(gw, h[3:], c2, s2)
    assert np.array_equal(a[0], np.concatenate([b1[0], b2[0]]))
    assert np.array_equal(ss_a, s2)


def test_conv_state_holds_the_last_inputs(orc):
    """After T >= d_conv - 1 tokens the conv state is the last d_conv - 1 rows
    of the qkv projection (the window's tail), whatever it held before."""
    gw = GdnWeights(256, 64, 2, 4, 4, (Q8_0,) * 5, 5, orc)
    h = np.random.default_rng(6).standard_normal((6, 256)).astype(np.float32)
    cs, ss = gw.fresh_state(np.random.default_rng(7))
    gdn_seg_restated(gw, h, cs, ss, orc)
    cur = orc.rms_norm_mul(h, gw.attn_norm, 1e-6)
    qkv = orc.mul_mat_id(Q8_0, 256, gw.conv_ch, 1, gw.w_qkv, cur[:, None, :], np.zeros((6, 1), np.int32))[:, 0, :]
    assert np.array_equal(cs, qkv[-3:].T)


def test_ggml_catches_a_perturbed_decay(orc, ref):
    """The comparison is sensitive to the recurrence's decay: the restatement fed
    decay rates (ssm_a) 0.1 % off fails the 1e-5 bar against ggml."""
    gw = GdnWeights(256, 64, 2, 4, 4, (Q8_0,) * 5, 9, orc)
    h = np.random.default_rng(8).standard_normal((4, 256)).astype(np.float32)
    cs, ss = gw.fresh_state(np.random.default_rng(9))
    want = ref.gdn_seg(gw, h, cs.copy(), ss.copy())[2]
    gw_bad = GdnWeights(256, 64, 2, 4, 4, (Q8_0,) * 5, 9, orc)
    gw_bad.ssm_a = (gw.ssm_a * 1.001).astype(np.float32)   # a slightly different decay rate
    got = gdn_seg_restated(gw_bad, h, cs.copy(), ss.copy(), orc)[2]
    assert rel(want, got) > 1e-5
