"""CPU checks of the attention half of Seg A (core/runtime.cpp:1976-2030,
build_attn 681-734): the numpy restatement in oracle_lib (attn_seg_restated)
against the reference ggml graph compiled from /root/reference
(oracle/_ref, qwref_attn_seg), plus what the mathematics fixes.

* restatement vs ggml: the roped Q within 1e-5 of its magnitude, attn_resid
  and ffn_in within 2e-4, the attention output within 1e-3 (a K element or a
  probability that lies at an f16 rounding boundary may round to the
  neighbouring f16 in one of them: one f16 step of a probability near 1/2 is
  ~2.4e-4 of a value), the V cache rows bit for bit and the K cache rows within
  one f16 step, at decode (T = 1, n_past 0 and 37), for a T = 5 batch after 11
  cached tokens (the causal mask inside the batch) and for a T = 64 chunk;
* one cached key: softmax is 1, so each head's output is its kv head's
  f16 V row (ggml's graph and the restatement);
* a planted mistake (the causal mask shifted by one key) is caught.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle_lib import AttnWeights, Oracle, Q4_K, Q6_K, RefGGML, attn_seg_restated, have_ref

H, NH, NKV, D = 512, 8, 2, 128
TYPES = (Q4_K, Q4_K, Q6_K, Q4_K)


def rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.fixture(scope="module")
def orc():
    return Oracle()


@pytest.fixture(scope="module")
def ref():
    if not have_ref():
        pytest.skip("oracle/_ref not built")
    return RefGGML()


def caches(n_ctx, n_fill, seed):
    rng = np.random.default_rng(seed)
    kc = np.zeros((n_ctx, NKV * D), np.uint16)
    vc = np.zeros((n_ctx, NKV * D), np.uint16)
    kc[:n_fill] = (rng.standard_normal((n_fill, NKV * D)) * 0.5).astype(np.float16).view(np.uint16)
    vc[:n_fill] = (rng.standard_normal((n_fill, NKV * D)) * 0.5).astype(np.float16).view(np.uint16)
    return kc, vc


@pytest.mark.parametrize("T,n_past", [(1, 0), (1, 37), (5, 11), (64, 100)])
def test_restatement_matches_reference_graph(orc, ref, T, n_past):
    aw = AttnWeights(H, NH, NKV, D, TYPES, seed=40 + T + n_past, oracle=orc)
    h = np.random.default_rng(T * 100 + n_past).standard_normal((T, H)).astype(np.float32)
    kc, vc = caches(256, n_past, seed=n_past)
    kc2, vc2 = kc.copy(), vc.copy()
    r_res, r_fin, r_q, r_att = ref.attn_seg(aw, h, n_past, kc, vc)
    o_res, o_fin, o_q, o_att = attn_seg_restated(aw, h, n_past, kc2, vc2, orc)
    assert rel(o_q, r_q) < 1e-5
    assert rel(o_att, r_att) < 1e-3
    assert rel(o_res, r_res) < 2e-4
    assert rel(o_fin, r_fin) < 2e-4
    assert np.array_equal(vc2, vc)
    dk = np.abs(kc2.view(np.float16).astype(np.float64) - kc.view(np.float16).astype(np.float64))
    ulp = np.spacing(np.abs(kc.view(np.float16))).astype(np.float64)
    assert np.all(dk <= ulp)
    assert np.array_equal(kc2[:n_past], kc[:n_past]) and not np.any(kc[n_past + T:])


def test_one_key_attention_is_the_value_row(orc, ref):
    aw = AttnWeights(H, NH, NKV, D, TYPES, seed=77, oracle=orc)
    h = np.random.default_rng(7).standard_normal((1, H)).astype(np.float32)
    kc, vc = caches(8, 0, seed=1)
    _, _, _, att = ref.attn_seg(aw, h, 0, kc, vc)
    v = vc[0].view(np.float16).astype(np.float32).reshape(NKV, D)
    want = np.repeat(v, NH // NKV, axis=0).reshape(-1)
    assert np.array_equal(att[0], want)
    kc2, vc2 = caches(8, 0, seed=1)
    _, _, _, att2 = attn_seg_restated(aw, h, 0, kc2, vc2, orc)
    assert np.array_equal(att2[0], want)


def test_planted_mask_shift_is_caught(orc, ref):
    """A copy of the restatement that lets every token see one key too many
    must disagree with the reference on a T > 1 batch."""
    aw = AttnWeights(H, NH, NKV, D, TYPES, seed=5, oracle=orc)
    h = np.random.default_rng(5).standard_normal((4, H)).astype(np.float32)
    kc, vc = caches(32, 6, seed=2)
    r_res, _, _, r_att = ref.attn_seg(aw, h, 6, kc.copy(), vc.copy())
    bad_kc, bad_vc = kc.copy(), vc.copy()
    _, _, _, att = attn_seg_restated(aw, h, 7, bad_kc, bad_vc, orc)   # (positions and mask one step late)
    assert rel(att, r_att) > 1e-2
