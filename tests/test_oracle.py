"""CPU tests that pin the oracle (oracle/qwmoe_oracle.cpp).

Three independent anchors:
  * golden fixtures written by the real ggml CPU backend (tests/golden/);
  * the real ggml CPU backend itself, compiled from /root/reference
    (oracle/_ref/libqwref.so) -- skipped where it is not built;
  * mathematics: exact integer identities, IEEE conversions checked against
    numpy, float64 references with stated error bounds, brute force.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest

from oracle_lib import (Q4_K, Q6_K, Q8_0, Q8_K, LayerWeights, Oracle, RefGGML, have_ref, row_size,
                        vec_dot_type)

GOLD = Path(__file__).resolve().parent / "golden" / "ggml_cpu_golden.npz"


@pytest.fixture(scope="module")
def orc():
    return Oracle()


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------- golden vectors

@pytest.mark.parametrize("t,name", [(Q8_0, "q8_0"), (Q4_K, "q4_K"), (Q6_K, "q6_K")])
def test_weight_quantizers_match_golden(orc, gold, t, name):
    X = gold["wq_x"]
    assert np.array_equal(orc.quantize(t, X).reshape(X.shape[0], -1), gold[f"wq_{name}"])


@pytest.mark.parametrize("t,name", [(Q8_0, "q8_0"), (Q8_K, "q8_K")])
def test_activation_quantizers_match_golden(orc, gold, t, name):
    X = gold["aq_x"]
    got = np.stack([orc.from_float(t, r) for r in X])
    assert np.array_equal(got, gold[f"aq_{name}"])


@pytest.mark.parametrize("t,name,K", [(Q4_K, "q4_K", 2048), (Q6_K, "q6_K", 1536), (Q8_0, "q8_0", 2048)])
def test_block_dots_match_golden(orc, gold, t, name, K):
    w, x, s = gold[f"dot_{name}_w"], gold[f"dot_{name}_x"], gold[f"dot_{name}_s"]
    got = np.array([orc.vec_dot(t, K, w[i], x[i]) for i in range(len(s))], np.float32)
    assert np.array_equal(bits(got), bits(s))


def test_float_ops_match_golden(orc, gold):
    assert np.array_equal(bits(orc.soft_max(gold["softmax_x"])), bits(gold["softmax_y"]))
    assert np.array_equal(orc.argsort_desc(gold["softmax_y"]), gold["argsort_y"])
    assert np.array_equal(bits(orc.swiglu(gold["swiglu_g"], gold["swiglu_u"])), bits(gold["swiglu_y"]))
    assert np.array_equal(bits(orc.rms_norm(gold["rms_x"], 1e-6)), bits(gold["rms_y"]))
    A, b = gold["dotf32_a"], gold["dotf32_b"]
    assert np.array_equal(bits([orc.vec_dot_f32(r, b) for r in A]), bits(gold["dotf32_y"]))
    A, b = gold["dotf32k_a"], gold["dotf32k_b"]
    assert np.array_equal(bits([orc.vec_dot_f32(r, b) for r in A]), bits(gold["dotf32k_y"]))


@pytest.mark.parametrize("name", ["l_q4k", "l_q80", "l_mix"])
def test_layers_match_golden(orc, gold, name):
    H, E, k, F, tg, tu, td, seed = (int(v) for v in gold[f"{name}_shape"])
    lw = LayerWeights(H, E, k, F, tg, tu, td, seed=seed, oracle=orc)
    h = hashlib.sha256()
    for arr in (lw.router.view(np.uint8), lw.gate, lw.up, lw.down):
        h.update(arr.tobytes())
    assert np.array_equal(np.frombuffer(h.digest(), np.uint8), gold[f"{name}_sha256"]), "weights regenerate"
    for T in (1, 5):
        r = orc.moe_layer(lw, gold[f"{name}_T{T}_x"], rms_eps=1e-6)
        assert np.array_equal(r["ids"], gold[f"{name}_T{T}_ids"])
        for key in ("weights", "out", "xnext"):
            assert np.array_equal(bits(r[key]), bits(gold[f"{name}_T{T}_{key}"])), key


def test_grouping_matches_golden(orc, gold):
    cnt, off, rows = orc.group_by_expert(gold["group_ids"], 16)
    assert np.array_equal(cnt, gold["group_counts"])
    assert np.array_equal(off, gold["group_offsets"])
    assert np.array_equal(rows, gold["group_rows"])


# ---------------------------------------------------------------- real ggml

needs_ref = pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (needs /root/reference)")


@needs_ref
@pytest.mark.parametrize("t,K", [(Q8_0, 2048), (Q4_K, 2048), (Q6_K, 1536), (Q4_K, 768), (Q8_0, 768)])
def test_random_dots_match_ggml(orc, t, K):
    ref = RefGGML()
    rng = np.random.default_rng(K + t)
    for _ in range(50):
        w = (rng.standard_normal(K) * 0.02).astype(np.float32)
        x = (rng.standard_normal(K) * rng.uniform(0.01, 10)).astype(np.float32)
        wq, xq = orc.quantize(t, w), orc.from_float(vec_dot_type(t), x)
        assert np.array_equal(wq, ref.quantize(t, w))
        assert np.array_equal(xq[: len(xq)], ref.from_float(vec_dot_type(t), x))
        assert bits(orc.vec_dot(t, K, wq, xq)) == bits(ref.vec_dot(t, K, wq, xq))


@needs_ref
def test_vec_dot_f32_tail_matches_ggml(orc):
    """Every n % 32 residue: the tail's mul/add vs fma pattern is the compiler's."""
    ref = RefGGML()
    rng = np.random.default_rng(7)
    for n in list(range(1, 70)) + [2047, 2048, 2049]:
        A = rng.standard_normal((16, n)).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        assert np.array_equal(bits([orc.vec_dot_f32(r, b) for r in A]), bits(ref.unary(4, A, b))), n


@needs_ref
@pytest.mark.parametrize("T", [1, 3, 17])
def test_layer_matches_ggml_all_intermediates(orc, T):
    ref = RefGGML()
    lw = LayerWeights(512, 16, 4, 512, Q4_K, Q4_K, Q6_K, seed=31, oracle=orc)
    x = np.random.default_rng(T).standard_normal((T, 512)).astype(np.float32)
    a, b = orc.moe_layer(lw, x, rms_eps=1e-6), ref.layer(lw, T, rms_eps=1e-6)(x)
    assert np.array_equal(a["ids"], b["ids"])
    for key in ("weights", "gate", "up", "act", "experts", "out", "xnext"):
        assert np.array_equal(bits(a[key]), bits(b[key])), key


@needs_ref
def test_stack_run_avx2_bit_exact_and_avx512_within_tolerance(orc):
    """The chained-stack driver the benchmark times: the AVX2 build equals the
    restatement bit for bit through a 4-layer stack (ids, output); the AVX-512
    build (the timed CPU baseline) takes the AVX-512 branch, and teacher-forced
    per layer its ids agree and its output stays far inside 1e-3."""
    from oracle_lib import REF_SO_AVX512, have_ref_avx512
    lws = [LayerWeights(1024, 32, 8, 512, Q4_K, Q4_K, Q4_K, seed=70 + l, oracle=orc) for l in range(4)]
    xs = np.random.default_rng(8).standard_normal((5, 1024)).astype(np.float32)
    ref = RefGGML()
    assert ref.isa() == 256
    L2 = [ref.layer(lw, 1, rms_eps=1e-6, n_threads=2) for lw in lws]
    r = ref.stack_run(L2, xs, 2, 2)
    assert r["step_s"].shape == (3,) and (r["step_s"] > 0).all()
    for s in range(3):
        x = xs[2 + s:3 + s]
        for l, lw in enumerate(lws):
            o = orc.moe_layer(lw, x, rms_eps=1e-6)
            assert np.array_equal(r["ids"][s, l], o["ids"][0])
            p = np.sort(L2[l](x)["probs"][0])[::-1]
            assert r["margin"][s, l] == p[7] - p[8]
            x = o["xnext"]
        assert np.array_equal(r["out"][s].view(np.int32), o["out"][0].view(np.int32))
    if not have_ref_avx512():
        pytest.skip("AVX-512 reference build or host ISA absent")
    r5 = RefGGML(REF_SO_AVX512)
    assert r5.isa() == 512
    L5 = [r5.layer(lw, 1, rms_eps=1e-6, n_threads=2) for lw in lws]
    for s in range(3):
        x = xs[2 + s:3 + s]
        for l, lw in enumerate(lws):
            o, c = orc.moe_layer(lw, x, rms_eps=1e-6), L5[l](x)
            assert np.array_equal(c["ids"][0], o["ids"][0])
            assert np.abs(c["out"] - o["out"]).max() <= 1e-5 * np.abs(o["out"]).max()
            x = o["xnext"]


@needs_ref
@pytest.mark.parametrize("T,n_res", [(1, 40), (1, 8), (3, 64), (5, 128)])
def test_router_resident_matches_ggml(orc, T, n_res):
    """Resident-only routing (core/runtime.cpp:870-881) against ggml's graph of
    the same ops: want = argsort_top_k(raw logits), then logits + mask (0 for
    the n_res resident experts, -inf else) before soft_max / top-k / weights.
    ids, weights, want and probabilities bit for bit; no absent expert is ever
    picked; with every expert resident the ids equal the unmasked router's and
    want equals them (softmax keeps the order)."""
    rng = np.random.default_rng(T * 100 + n_res)
    E, H, k = 128, 256, 8
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    res = np.sort(rng.choice(E, n_res, replace=False))
    mask = np.full(E, -np.inf, np.float32)
    mask[res] = 0.0
    ids, w, want, probs = orc.router_resident(W, x, k, mask)
    rids, rw, rwant, rprobs = RefGGML().router_resident(W, x, k, mask)
    assert np.array_equal(ids, rids)
    assert np.array_equal(want, rwant)
    assert np.array_equal(w.view(np.int32), rw.view(np.int32))
    assert np.array_equal(probs.view(np.int32), rprobs.view(np.int32))
    assert np.isin(ids, res).all()
    assert np.all(probs[:, np.setdiff1d(np.arange(E), res)] == 0.0)
    pids, pw, logits, _ = orc.router(W, x, k)
    assert np.array_equal(want, np.argsort(-logits, axis=1, kind="stable")[:, :k])   # no ties in random logits
    if n_res == E:
        assert np.array_equal(ids, pids) and np.array_equal(want, pids)
        assert np.array_equal(w.view(np.int32), pw.view(np.int32))


@needs_ref
def test_rms_norm_mul_matches_ggml(orc):
    """The router input of a decoder layer: mul(rms_norm(x), w) bit for bit."""
    ref = RefGGML()
    rng = np.random.default_rng(41)
    for n, rows in ((2048, 3), (4096, 1), (512, 7)):
        x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
        w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        got = orc.rms_norm_mul(x, w, 1e-6)
        want = ref.unary(5, x, w, param=1e-6)
        assert np.array_equal(got.view(np.int32), want.view(np.int32)), (n, rows)
        assert not np.array_equal(got, orc.rms_norm(x, 1e-6))      # the weight is applied


@needs_ref
@pytest.mark.parametrize("types", [(Q4_K, Q4_K, Q4_K), (Q4_K, Q4_K, Q6_K), (Q8_0, Q8_0, Q8_0)])
@pytest.mark.parametrize("T", [1, 3])
def test_shared_expert_matches_ggml(orc, types, T):
    """The shared-expert branch (silu, mul, sigmoid gate, adds) bit for bit
    against the reference graph, with and without the residual add."""
    from oracle_lib import SharedWeights
    se = SharedWeights(1024, 512, *types, seed=60 + T, oracle=orc)
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, 1024)).astype(np.float32)
    mo = rng.standard_normal((T, 1024)).astype(np.float32)
    res = rng.standard_normal((T, 1024)).astype(np.float32)
    ref = RefGGML()
    for resid in (None, res):
        got = orc.shared_expert_add(se, x, mo, resid)
        want = ref.shared_expert_add(se, x, mo, resid)
        assert np.array_equal(got.view(np.int32), want.view(np.int32))
    # the branch is not a no-op: its share moves the output
    assert np.abs(orc.shared_expert_add(se, x, mo) - mo).max() > 1e-3


@needs_ref
def test_mul_mat_id_matches_ggml(orc):
    ref = RefGGML()
    rng = np.random.default_rng(3)
    for t, K, N in ((Q4_K, 512, 96), (Q6_K, 768, 64), (Q8_0, 256, 80)):
        n_as, T, n_ids = 12, 7, 3
        w = orc.quantize(t, (rng.standard_normal((n_as * N, K)) * 0.02).astype(np.float32))
        b = rng.standard_normal((T, n_ids, K)).astype(np.float32)
        ids = np.stack([rng.choice(n_as, n_ids, replace=False) for _ in range(T)]).astype(np.int32)
        got = orc.mul_mat_id(t, K, N, n_as, w, b, ids)
        assert np.array_equal(bits(got), bits(ref.mul_mat_id(t, K, N, n_as, w, b, ids)))


# ---------------------------------------------------------------- mathematics

def test_fp16_conversion_is_ieee_rne(orc):
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08,
                  2.9802326e-08, 1e-10, 1.00048828125, 1.0009765625, 1.00146484375], np.float32),
    ]).astype(np.float32)
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([orc.lib.orc_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)
    hs = np.arange(0, 1 << 16, dtype=np.uint16)
    hs = hs[(hs & 0x7c00) != 0x7c00]
    back = np.array([orc.lib.orc_f16_to_f32(int(h)) for h in hs], np.float32)
    assert np.array_equal(bits(back), bits(hs.view(np.float16).astype(np.float32)))


def _unpack_q4k(q: np.ndarray, nb: int):
    """Brute-force field extraction of Q4_K blocks -> (d, dmin, sc[8], mn[8], q[256])."""
    blk = q.reshape(nb, 144)
    d = blk[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float64)
    dmin = blk[:, 2:4].copy().view(np.float16)[:, 0].astype(np.float64)
    s = blk[:, 4:16].astype(np.int64)
    sc = np.zeros((nb, 8), np.int64)
    mn = np.zeros((nb, 8), np.int64)
    for j in range(8):
        if j < 4:
            sc[:, j] = s[:, j] & 63
            mn[:, j] = s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
            mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    qs = blk[:, 16:].astype(np.int64)
    vals = np.zeros((nb, 256), np.int64)
    for c in range(4):
        vals[:, 64 * c: 64 * c + 32] = qs[:, 32 * c: 32 * c + 32] & 0xF
        vals[:, 64 * c + 32: 64 * c + 64] = qs[:, 32 * c: 32 * c + 32] >> 4
    return d, dmin, sc, mn, vals


def _unpack_q8k(y: np.ndarray, nb: int):
    blk = y.reshape(nb, 292)
    d = blk[:, 0:4].copy().view(np.float32)[:, 0].astype(np.float64)
    qs = blk[:, 4:260].copy().view(np.int8).astype(np.int64)
    bs = blk[:, 260:292].copy().view(np.int16).astype(np.int64)
    return d, qs, bs


def test_q4k_dot_integer_identity(orc):
    """sum_n sumi[n] == sum_l sc(l) q(l) q8(l) and sum_i prod[i] == sum_l mn(l) q8(l),
    computed here by plain unpacking (no lane partition); the float result then
    equals d_y*(d*sumi - dmin*summ) to within the fp32 accumulation bound."""
    rng = np.random.default_rng(11)
    K = 2048
    nb = K // 256
    for _ in range(20):
        wq = orc.quantize(Q4_K, (rng.standard_normal(K) * 0.02).astype(np.float32))
        yq = orc.from_float(Q8_K, rng.standard_normal(K).astype(np.float32))
        lanes, mins = orc.dot_lanes(Q4_K, K, wq, yq)
        d, dmin, sc, mn, q = _unpack_q4k(wq, nb)
        dy, q8, bs = _unpack_q8k(yq, nb)
        sub = np.arange(256) // 32
        sumi = (sc[:, sub] * q * q8).sum(1)
        summ = (mn[:, sub] * q8).sum(1)
        assert np.array_equal(lanes.sum(1), sumi)
        assert np.array_equal(mins.sum(1), summ)
        assert np.array_equal(bs, q8.reshape(nb, 16, 16).sum(2))        # bsums are group sums
        exact = float((dy * (d * sumi - dmin * summ)).sum())
        got = float(orc.vec_dot(Q4_K, K, wq, yq))
        scale = float((np.abs(dy * d * sumi) + np.abs(dy * dmin * summ)).sum())
        assert abs(got - exact) <= 64 * np.finfo(np.float32).eps * scale


def test_q6k_and_q8_0_dot_integer_identity(orc):
    rng = np.random.default_rng(12)
    K = 1536
    nb = K // 256
    wq = orc.quantize(Q6_K, (rng.standard_normal(K) * 0.02).astype(np.float32))
    yq = orc.from_float(Q8_K, rng.standard_normal(K).astype(np.float32))
    lanes, _ = orc.dot_lanes(Q6_K, K, wq, yq)
    deq = orc.dequantize(Q6_K, wq, K).astype(np.float64)
    dy, q8, _ = _unpack_q8k(yq, nb)
    blk = wq.reshape(nb, 210)
    d = blk[:, 208:210].copy().view(np.float16)[:, 0].astype(np.float64)
    scs = blk[:, 192:208].copy().view(np.int8).astype(np.float64)
    # dequantized value = d * sc * (q - 32): integer part recovered exactly
    qint = np.rint(deq.reshape(nb, 256) / (d[:, None] * np.repeat(scs, 16, axis=1) + 1e-300))
    qint = np.where(np.repeat(scs, 16, axis=1) == 0, 0, qint)
    ref_sumi = (np.repeat(scs, 16, axis=1) * qint * q8).sum(1)
    assert np.array_equal(lanes.sum(1).astype(np.float64), ref_sumi)
    # Q8_0 x Q8_0: lanes are plain byte dots
    K = 256
    a = orc.quantize(Q8_0, (rng.standard_normal(K) * 0.02).astype(np.float32))
    b = orc.from_float(Q8_0, rng.standard_normal(K).astype(np.float32))
    lanes, _ = orc.dot_lanes(Q8_0, K, a, b)
    qa = a.reshape(-1, 34)[:, 2:].copy().view(np.int8).astype(np.int64)
    qb = b.reshape(-1, 34)[:, 2:].copy().view(np.int8).astype(np.int64)
    assert np.array_equal(lanes.sum(1), (qa * qb).sum(1))


def test_q8k_quantizer_properties(orc):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(4096) * 3).astype(np.float32)
    d, qs, bs = _unpack_q8k(orc.from_float(Q8_K, x), 16)
    xb = x.reshape(16, 256).astype(np.float64)
    amax_idx = np.argmax(np.abs(xb), axis=1)               # first occurrence, like the reference
    assert np.all(qs[np.arange(16), amax_idx] == -127)     # the max maps to -127 (iscale = -127/max)
    assert np.all(np.abs(qs * d[:, None] - xb) <= np.abs(d)[:, None] * 0.5000001)
    assert np.array_equal(bs, qs.reshape(16, 16, 16).sum(2))


def test_nearest_int_is_round_half_even(orc):
    # through Q8_K: max = -127 gives iscale = -127/max = 1, so q = nearest_int(x)
    x = np.zeros(256, np.float32)
    x[0] = -127.0
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5]
    _, qs, _ = _unpack_q8k(orc.from_float(Q8_K, x), 1)
    assert list(qs[0, :9]) == list(np.rint(x[:9]).astype(int))       # numpy rint is half-to-even
    assert list(qs[0, 1:9]) == [0, 2, 2, 0, -2, -2, 4, 126]


def test_softmax_and_expf_accuracy(orc):
    rng = np.random.default_rng(9)
    xs = rng.uniform(-100, 0, 20000).astype(np.float32)
    got = np.array([orc.lib.orc_v_expf(float(v)) for v in xs], np.float64)
    want = np.exp(xs.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - want) / ulp) < 2.0           # ggml documents 1.45 ulp + 0.5
    L = (rng.standard_normal((16, 128)) * 2).astype(np.float32)
    p = orc.soft_max(L)
    p64 = np.exp(L - L.max(1, keepdims=True).astype(np.float64))
    p64 /= p64.sum(1, keepdims=True)
    assert np.max(np.abs(p - p64) / p64) < 1e-5
    assert np.allclose(p.sum(1), 1.0, atol=1e-5)


def test_v_expf_never_increases_as_x_decreases(orc):
    """Every float in [-inf, -0]: a smaller x never gets a larger ggml_v_expf.
    The GPU router posts its top-k from this (with a margin that rounding of
    e * (1/sum) cannot undo) before the softmax sums are formed."""
    from concurrent.futures import ThreadPoolExecutor
    edges = [0x80000000 + ((0xFF800000 - 0x80000000) * i) // 8 for i in range(9)]   # chunks share end points
    with ThreadPoolExecutor(8) as ex:                  # ctypes drops the GIL during the call
        bad = list(ex.map(lambda i: orc.lib.orc_v_expf_increases(edges[i], edges[i + 1]), range(8)))
    assert bad == [0] * 8
    assert orc.lib.orc_v_expf(-0.0) == 1.0 and orc.lib.orc_v_expf(float("-inf")) == 0.0
    # the counter sees increases where they exist: x = 1.0 upward, 256 steps
    assert orc.lib.orc_v_expf_increases(0x3F800000, 0x3F800100) > 200


def test_argsort_brute_force_without_ties(orc):
    rng = np.random.default_rng(2)
    x = rng.permutation(np.arange(128, dtype=np.float32)).reshape(1, 128) / 7
    assert np.array_equal(orc.argsort_desc(x)[0], np.argsort(-x[0], kind="stable"))


def test_rms_norm_and_swiglu_vs_float64(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 2048)).astype(np.float32)
    y = orc.rms_norm(x, 1e-6)
    x64 = x.astype(np.float64)
    y64 = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6)
    assert np.max(np.abs(y - y64)) < 1e-5
    g = (rng.standard_normal((4, 768)) * 3).astype(np.float32)
    u = rng.standard_normal((4, 768)).astype(np.float32)
    s = orc.swiglu(g, u)
    g64 = g.astype(np.float64)
    s64 = g64 / (1 + np.exp(-g64)) * u
    assert np.max(np.abs(s - s64) / (np.abs(s64) + 1e-30)) < 2e-6


def test_mul_mat_id_vs_dequantized_float64(orc):
    """dst == dequant(W) . dequant(quant(b)) up to fp32 accumulation error."""
    rng = np.random.default_rng(6)
    for t, K, N in ((Q4_K, 512, 32), (Q6_K, 512, 32), (Q8_0, 512, 32)):
        n_as, T, n_ids = 5, 3, 2
        w = orc.quantize(t, (rng.standard_normal((n_as * N, K)) * 0.02).astype(np.float32))
        b = rng.standard_normal((T, 1, K)).astype(np.float32)
        ids = np.array([[0, 3], [4, 1], [2, 0]], np.int32)
        got = orc.mul_mat_id(t, K, N, n_as, w, b, ids)
        W = orc.dequantize(t, w, n_as * N * K).reshape(n_as, N, K).astype(np.float64)
        vdt = vec_dot_type(t)
        for tt in range(T):
            xb = orc.dequantize(Q8_0, orc.from_float(Q8_0, b[tt, 0]), K) if vdt == Q8_0 else None
            if vdt == Q8_K:
                d, qs, _ = _unpack_q8k(orc.from_float(Q8_K, b[tt, 0]), K // 256)
                xb = (qs * d[:, None]).reshape(-1)
            for e in range(n_ids):
                want = W[ids[tt, e]] @ xb.astype(np.float64)
                assert np.max(np.abs(got[tt, e] - want)) < 1e-4 * (np.abs(W[ids[tt, e]]) @ np.abs(xb)).max()


def test_grouping_is_stable_counting_sort(orc):
    rng = np.random.default_rng(8)
    ids = np.stack([rng.choice(40, 6, replace=False) for _ in range(33)]).astype(np.int32)
    cnt, off, rows = orc.group_by_expert(ids, 40)
    assert np.array_equal(cnt, np.bincount(ids.reshape(-1), minlength=40))
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")                 # stable sort by expert over (t, e) order
    assert np.array_equal(rows[:, 1] * 6 + rows[:, 0], order)
    assert np.array_equal(off[:-1], np.concatenate([[0], np.cumsum(cnt)[:-1]]))


def test_slot_permutation_roundtrip(orc):
    """Reading experts through a permuted pool equals reading the dense tensor."""
    lw_d = LayerWeights(256, 8, 2, 256, Q4_K, Q4_K, Q4_K, seed=21, oracle=orc)
    lw_p = LayerWeights(256, 8, 2, 256, Q4_K, Q4_K, Q4_K, seed=21, oracle=orc, permute=True)
    x = np.random.default_rng(1).standard_normal((3, 256)).astype(np.float32)
    a, b = orc.moe_layer(lw_d, x), orc.moe_layer(lw_p, x)
    assert np.array_equal(a["ids"], b["ids"])
    assert np.array_equal(bits(a["out"]), bits(b["out"]))


def test_planted_mistakes_are_caught(orc, gold):
    """A wrong sign in the min term or a transposed lane assignment must fail the pins."""
    K = 2048
    w, x, s = gold["dot_q4_K_w"], gold["dot_q4_K_x"], gold["dot_q4_K_s"]
    lanes, mins = orc.dot_lanes(Q4_K, K, w[0], x[0])
    nb = K // 256
    dy, _, _ = _unpack_q8k(x[0], nb)
    d, dmin, *_ = _unpack_q4k(w[0], nb)
    # correct closed form reproduces the golden value to fp32 accuracy; a flipped min sign does not
    good = float((dy * (d * lanes.sum(1) - dmin * mins.sum(1))).sum())
    bad = float((dy * (d * lanes.sum(1) + dmin * mins.sum(1))).sum())
    assert abs(good - s[0]) < 1e-4 * abs(s).max()
    assert abs(bad - s[0]) > 1e-3 * abs(s).max()
