"""GPU parity: every HIP kernel against the CPU oracle, through the C ABI.

Bar: bit-exact for integers and bytes (ids, grouping, quantized blocks) and
for the fp32 outputs too -- the kernels replay the reference CPU float order,
so every comparison below is on bit patterns.  The one documented exception is
RMSNorm (double-precision sum in a different order; see test_rms_norm).
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from questwend_amd import ops  # noqa: E402
from oracle_lib import (Q4_K, Q6_K, Q8_0, Q8_K, LayerWeights, Oracle, row_size,  # noqa: E402
                        vec_dot_type)

GOLD = Path(__file__).resolve().parent / "golden" / "ggml_cpu_golden.npz"
DEV = "cuda:0"


def note(msg: str) -> None:
    print(f"[gpu-parity] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    prev = ops.set_mfma_min_rows(0)   # every expert on the bit-exact GEMV (the matrix cores: test_gpu_prefill.py)
    yield
    torch.cuda.synchronize()
    ops.set_mfma_min_rows(prev)


@pytest.fixture(scope="module")
def orc():
    return Oracle()


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def assert_status_clean():
    st = ops.device_status(clear=True)
    assert st & (qa.STATUS_BAD_ID | qa.STATUS_BAD_SLOT) == 0, f"device status {st}"


# ---------------------------------------------------------------- quantizers

@pytest.mark.parametrize("t,name", [(Q8_0, "q8_0"), (Q8_K, "q8_K")])
def test_activation_quantizers(orc, gold, t, name):
    note(f"activation quantizer {name}")
    X = gold["aq_x"]
    got = host(ops.quantize_act(t, dev(X)))
    assert np.array_equal(got, gold[f"aq_{name}"])
    rng = np.random.default_rng(1)
    Y = (rng.standard_normal((64, 2048)) * rng.uniform(1e-3, 1e3, (64, 1))).astype(np.float32)
    got = host(ops.quantize_act(t, dev(Y)))
    want = np.stack([orc.from_float(t, r) for r in Y])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("t,name", [(Q8_0, "q8_0"), (Q4_K, "q4_K"), (Q6_K, "q6_K")])
def test_weight_quantizers(orc, gold, t, name):
    note(f"weight quantizer {name}")
    X = gold["wq_x"]
    got = host(ops.quantize_chunk(t, dev(X)))
    assert np.array_equal(got, gold[f"wq_{name}"])
    rng = np.random.default_rng(2)
    W = (rng.standard_normal((96, 1536)) * 0.02).astype(np.float32)
    assert np.array_equal(host(ops.quantize_chunk(t, dev(W))).reshape(-1), orc.quantize(t, W))


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K])
def test_dequantize(orc, t):
    note(f"dequantize {t}")
    rng = np.random.default_rng(3)
    q = orc.quantize(t, (rng.standard_normal(4096) * 0.02).astype(np.float32))
    assert np.array_equal(bits(host(ops.dequantize(t, dev(q), 4096))), bits(orc.dequantize(t, q, 4096)))


# ---------------------------------------------------------------- mul_mat_id

def _mmid_case(orc, t, K, N, n_as, T, n_ids, ne11, seed, permute=False, strided_ids=False):
    rng = np.random.default_rng(seed)
    w = orc.quantize(t, (rng.standard_normal((n_as * N, K)) * 0.02).astype(np.float32))
    b = rng.standard_normal((T, ne11, K)).astype(np.float32)
    ids = np.stack([rng.choice(n_as, n_ids, replace=False) for _ in range(T)]).astype(np.int32)
    slot_of = None
    w_used = w
    if permute:
        perm = rng.permutation(n_as).astype(np.int32)
        pool = np.empty_like(w.reshape(n_as, -1))
        pool[perm] = w.reshape(n_as, -1)
        w_used, slot_of = pool.reshape(-1), perm
    want = orc.mul_mat_id(t, K, N, n_as, w, b, ids)
    ids_d = dev(ids)
    if strided_ids:  # the strided view argsort_top_k hands over: [T, n_as] buffer, first n_ids columns
        big = np.full((T, n_as), -7, np.int32)
        big[:, :n_ids] = ids
        ids_d = dev(big)[:, :n_ids]
    got = ops.mul_mat_id(t, dev(w_used), K, N, n_as, dev(b), ids_d,
                         slot_of=None if slot_of is None else dev(slot_of))
    return host(got), want


@pytest.mark.parametrize("t,K,N", [(Q4_K, 2048, 256), (Q4_K, 768, 512), (Q8_0, 2048, 256), (Q8_0, 768, 512),
                                   (Q6_K, 1536, 128), (Q4_K, 4096, 64)])
@pytest.mark.parametrize("T,n_ids,ne11", [(1, 8, 1), (5, 8, 8), (33, 4, 1)])
def test_mul_mat_id_bit_exact(orc, t, K, N, T, n_ids, ne11):
    note(f"mul_mat_id type={t} K={K} N={N} T={T} n_ids={n_ids} ne11={ne11}")
    n_as = 12
    got, want = _mmid_case(orc, t, K, N, n_as, T, n_ids, ne11, seed=K + N + T)
    assert np.array_equal(bits(got), bits(want))
    assert_status_clean()


def test_mul_mat_id_slot_table_and_strided_ids(orc):
    note("mul_mat_id through a permuted slot pool with strided ids")
    got, want = _mmid_case(orc, Q4_K, 1024, 256, 24, 7, 6, 1, seed=5, permute=True, strided_ids=True)
    assert np.array_equal(bits(got), bits(want))
    assert_status_clean()


def test_mul_mat_id_ragged_rows(orc):
    note("mul_mat_id N not a multiple of the row tile, many tokens on one expert")
    rng = np.random.default_rng(9)
    t, K, N, n_as, T = Q4_K, 512, 70, 6, 40
    w = orc.quantize(t, (rng.standard_normal((n_as * N, K)) * 0.02).astype(np.float32))
    b = rng.standard_normal((T, 1, K)).astype(np.float32)
    ids = np.stack([[0, 1 + (i % 5)] for i in range(T)]).astype(np.int32)  # expert 0 takes every token
    got = host(ops.mul_mat_id(t, dev(w), K, N, n_as, dev(b), dev(ids)))
    assert np.array_equal(bits(got), bits(orc.mul_mat_id(t, K, N, n_as, w, b, ids)))


@pytest.mark.parametrize("t,K", [(Q4_K, 4096), (Q4_K, 768), (Q6_K, 1536), (Q6_K, 512)])
@pytest.mark.parametrize("off", [0, 2, 4, 5])
def test_mul_mat_id_small_bins_unaligned_ragged(orc, t, K, off):
    """Bins of at most eight rows (decode and verify batches) with N not a
    multiple of any row tile and the weights starting off bytes past an aligned
    address (rows then misaligned for word reads)."""
    note(f"mul_mat_id small bins type={t} K={K} N=70 weight offset {off}")
    rng = np.random.default_rng(K + off)
    N, n_as = 70, 9
    w = orc.quantize(t, (rng.standard_normal((n_as * N, K)) * 0.02).astype(np.float32))
    buf = np.zeros(w.size + 16, np.uint8)
    buf[off:off + w.size] = w
    wd = dev(buf)[off:off + w.size]
    for T, n_ids in ((1, 8), (3, 4), (8, 2)):
        b = rng.standard_normal((T, 1, K)).astype(np.float32)
        ids = np.stack([rng.choice(n_as, n_ids, replace=False) for _ in range(T)]).astype(np.int32)
        got = host(ops.mul_mat_id(t, wd, K, N, n_as, dev(b), dev(ids)))
        assert np.array_equal(bits(got), bits(orc.mul_mat_id(t, K, N, n_as, w, b, ids))), f"T={T}"
    assert_status_clean()


def test_mul_mat_id_bad_id_sets_status(orc):
    note("mul_mat_id with an out-of-range id (host-forced error path)")
    rng = np.random.default_rng(4)
    K, N, n_as = 256, 32, 4
    w = orc.quantize(Q4_K, (rng.standard_normal((n_as * N, K)) * 0.02).astype(np.float32))
    b = rng.standard_normal((1, 1, K)).astype(np.float32)
    ids = np.array([[1, 9]], np.int32)
    out = torch.full((1, 2, N), 123.0, device=DEV)
    ops.mul_mat_id(Q4_K, dev(w), K, N, n_as, dev(b), dev(ids), out=out)
    st = ops.device_status(clear=True)
    assert st & qa.STATUS_BAD_ID
    o = host(out)
    assert np.all(o[0, 1] == 123.0)        # the bad pair was skipped, not written
    want = orc.mul_mat_id(Q4_K, K, N, n_as, w, b, np.array([[1, 0]], np.int32))
    assert np.array_equal(bits(o[0, 0]), bits(want[0, 0]))


# ---------------------------------------------------------------- grouping

@pytest.mark.parametrize("T,k,n_as,dup", [(1, 8, 128, False), (5, 8, 128, False), (512, 8, 128, False),
                                          (1024, 8, 128, False), (4096, 8, 128, False), (3, 2, 5000, False),
                                          (700, 6, 1500, False), (333, 7, 3, True), (257, 5, 64, True)])
def test_group_by_expert(orc, T, k, n_as, dup):
    """Stable grouping (token outer, slot inner) bit-exact; dup routes one token to
    the same matrix several times, as ggml_mul_mat_id allows, so one 64-pair chunk
    holds long runs of equal keys; n_as above 1024 keeps the counters in global memory."""
    note(f"group_by_expert T={T} k={k} n_as={n_as} dup={dup}")
    rng = np.random.default_rng(T + n_as)
    p = np.arange(1, n_as + 1, dtype=np.float64) ** -1.1
    p /= p.sum()
    ids = np.stack([rng.choice(n_as, k, replace=dup, p=p) for _ in range(T)]).astype(np.int32)
    cnt, off, rows = (host(x) for x in ops.group_by_expert(dev(ids), n_as))
    c2, o2, r2 = orc.group_by_expert(ids, n_as)
    assert np.array_equal(cnt, c2)
    assert np.array_equal(off, o2)
    assert np.array_equal(rows, r2)


# ---------------------------------------------------------------- router

@pytest.mark.parametrize("H,E,k,T", [(2048, 128, 8, 1), (2048, 128, 8, 5), (4096, 128, 8, 3), (2048, 128, 8, 64),
                                     (512, 16, 4, 9), (2052, 64, 6, 2), (8192, 64, 4, 2),
                                     # T > 16 (the tiled logits kernel): partial expert and token tiles, H tails
                                     (1004, 24, 3, 70), (2052, 64, 6, 37), (4096, 128, 8, 100),
                                     # T > 16, H % 512 == 0, E % 16 == 0 (the LDS-staged logits kernel):
                                     # one or more chunks, partial token tiles
                                     (512, 32, 4, 33), (2048, 48, 6, 20)])
def test_router_bit_exact(orc, H, E, k, T):
    note(f"router H={H} E={E} k={k} T={T}")
    rng = np.random.default_rng(H + E + T)
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids, w, probs = ops.router_topk(dev(W), dev(x), k, want_probs=True)
    i2, w2, _, p2 = orc.router(W, x, k)
    assert np.array_equal(host(ids), i2)
    assert np.array_equal(bits(host(w)), bits(w2))
    assert np.array_equal(bits(host(probs)), bits(p2))


def test_router_ties_replay_std_sort(orc):
    """Duplicated router rows give exactly equal probabilities inside the top-k."""
    note("router with exact probability ties")
    rng = np.random.default_rng(17)
    H, E, k, T = 2048, 128, 8, 16
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    _, _, logits, _ = orc.router(W, x, k)
    for t in range(T):  # copy the best expert's row of this token onto a few others
        top = int(np.argmax(logits[t]))
        for j in rng.choice(E, 3, replace=False):
            W[j] = W[top]
    ops.device_status(clear=True)
    ids, w = ops.router_topk(dev(W), dev(x), k)
    i2, w2, _, _ = orc.router(W, x, k)
    assert np.array_equal(host(ids), i2)
    assert np.array_equal(bits(host(w)), bits(w2))
    assert ops.device_status(clear=True) & qa.STATUS_TOPK_TIE_SORT


def test_router_non_finite_input(orc):
    """A NaN or +Inf in a token's input makes every logit of that token
    non-finite and softmax makes every probability NaN; std::sort then sees
    all-equivalent values, and the replay must give its permutation (the other
    tokens are unaffected)."""
    note("router with NaN / +Inf inputs")
    rng = np.random.default_rng(23)
    H, E, k, T = 512, 64, 6, 4
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    x[1, 7] = np.nan
    x[3, 100] = np.inf
    ops.device_status(clear=True)
    ids, w, probs = ops.router_topk(dev(W), dev(x), k, want_probs=True)
    i2, w2, _, p2 = orc.router(W, x, k)
    ids, w, probs = host(ids), host(w), host(probs)
    for t in (0, 2):
        assert np.array_equal(ids[t], i2[t])
        assert np.array_equal(bits(w[t]), bits(w2[t]))
    want = np.empty(E, np.int32)
    qa.lib().qwmoe_host_argsort_desc(np.full(E, np.nan, np.float32).ctypes.data, E, want.ctypes.data)
    for t in (1, 3):
        assert np.isnan(probs[t]).all() and np.isnan(p2[t]).all()
        assert np.array_equal(ids[t], want[:k]) and np.array_equal(i2[t], want[:k]), f"token {t}"
        assert np.isnan(w[t]).all()
    assert ops.device_status(clear=True) == qa.STATUS_TOPK_TIE_SORT


# ---------------------------------------------------------------- FFN tail

def test_swiglu_and_weighted_sum(orc):
    note("swiglu / weighted sum")
    rng = np.random.default_rng(6)
    g = (rng.standard_normal((40, 768)) * 4).astype(np.float32)
    u = rng.standard_normal((40, 768)).astype(np.float32)
    assert np.array_equal(bits(host(ops.swiglu(dev(g), dev(u)))), bits(orc.swiglu(g, u)))
    for T, k in ((1, 8), (1, 3), (1, 40), (5, 8)):
        ex = rng.standard_normal((T, k, 2048)).astype(np.float32)
        wts = rng.uniform(0, 1, (T, k)).astype(np.float32)
        got = host(ops.weighted_sum(dev(ex), dev(wts)))
        if T == 1:
            want = np.array([orc.vec_dot_f32(ex[0, :, h], wts[0]) for h in range(2048)], np.float32)[None]
        else:
            want = np.zeros((T, 2048), np.float32)
            for t in range(T):
                acc = ex[t, 0] * wts[t, 0]
                for i in range(1, k):
                    acc = (acc + ex[t, i] * wts[t, i]).astype(np.float32)
                want[t] = acc
        assert np.array_equal(bits(got), bits(want)), (T, k)


def test_rms_norm(orc):
    """The only non-bit-exact-by-construction op: the double sum is a tree here.
    Its result is rounded to float before use, so it still matches bit for bit
    except when the sum sits ~1e-13 from a float rounding boundary."""
    note("rms_norm")
    rng = np.random.default_rng(8)
    x = rng.standard_normal((256, 2048)).astype(np.float32)
    got = host(ops.rms_norm(dev(x), 1e-6))
    want = orc.rms_norm(x, 1e-6)
    mism = np.sum(np.any(bits(got) != bits(want), axis=1))
    assert mism == 0
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-6)) < 1e-6


# ---------------------------------------------------------------- full layer

def _layer_gpu(lw: LayerWeights):
    slots = None
    if lw.slot_of is not None:
        slots = tuple(dev(s) for s in lw.slot_of)
    tensors = [dev(lw.router), dev(lw.gate), dev(lw.up), dev(lw.down)]
    L = ops.make_layer(lw.H, lw.E, lw.k, lw.F, *tensors, (lw.type_gate, lw.type_up, lw.type_down),
                       n_slots=(lw.n_slots,) * 3, slots=slots)
    return L, tensors, slots


@pytest.mark.parametrize("name", ["l_q4k", "l_q80", "l_mix"])
def test_layer_golden(orc, gold, name):
    H, E, k, F, tg, tu, td, seed = (int(v) for v in gold[f"{name}_shape"])
    note(f"ffn_layer golden {name}")
    lw = LayerWeights(H, E, k, F, tg, tu, td, seed=seed, oracle=orc)
    h = hashlib.sha256()
    for arr in (lw.router.view(np.uint8), lw.gate, lw.up, lw.down):
        h.update(arr.tobytes())
    assert np.array_equal(np.frombuffer(h.digest(), np.uint8), gold[f"{name}_sha256"])
    L, keep, _ = _layer_gpu(lw)
    for T in (1, 5):
        out, xn, ids, w = ops.ffn_layer(L, dev(gold[f"{name}_T{T}_x"]), rms_eps=1e-6)
        assert np.array_equal(host(ids), gold[f"{name}_T{T}_ids"])
        assert np.array_equal(bits(host(w)), bits(gold[f"{name}_T{T}_weights"]))
        assert np.array_equal(bits(host(out)), bits(gold[f"{name}_T{T}_out"]))
        assert np.array_equal(bits(host(xn)), bits(gold[f"{name}_T{T}_xnext"]))
    assert_status_clean()


@pytest.mark.parametrize("types,T,permute", [((Q4_K,) * 3, 1, False), ((Q4_K,) * 3, 5, True),
                                             ((Q8_0,) * 3, 1, False), ((Q4_K, Q4_K, Q6_K), 3, True)])
def test_layer_30b_shape(orc, types, T, permute):
    """H=2048, F=768, k=8 at E=16 experts (oracle quantization time bounds E;
    the router needs E % 8 == 0)."""
    note(f"ffn_layer 30B shape types={types} T={T} permute={permute}")
    lw = LayerWeights(2048, 16, 8, 768, *types, seed=100 + T, oracle=orc, permute=permute)
    L, keep, _ = _layer_gpu(lw)
    x = np.random.default_rng(T).standard_normal((T, 2048)).astype(np.float32)
    out, xn, ids, w = ops.ffn_layer(L, dev(x), rms_eps=1e-6)
    r = orc.moe_layer(lw, x, rms_eps=1e-6)
    assert np.array_equal(host(ids), r["ids"])
    assert np.array_equal(bits(host(w)), bits(r["weights"]))
    assert np.array_equal(bits(host(out)), bits(r["out"]))
    assert np.array_equal(bits(host(xn)), bits(r["xnext"]))
    assert_status_clean()


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("off", [1, 2, 4])
@pytest.mark.parametrize("moved", ["gate", "up"])
def test_layer_gate_up_different_alignment(orc, t, off, moved):
    """ffn_layer launches gate and up as one pair: with one of them off bytes
    past an aligned address and the other aligned, the pair must take the loads
    that suit both (Q4_K direct loads need 16-byte rows, Q6_K 4-byte)."""
    note(f"ffn_layer type={t}: {moved} at byte offset {off}, the other aligned")
    lw = LayerWeights(2048, 16, 8, 768, t, t, Q4_K, seed=300 + off + t, oracle=orc)
    src = lw.gate if moved == "gate" else lw.up
    buf = torch.zeros(src.size + 64, dtype=torch.uint8, device=DEV)
    mv = buf[off:off + src.size]
    mv.copy_(dev(src))
    gate = mv if moved == "gate" else dev(lw.gate)
    up = mv if moved == "up" else dev(lw.up)
    keep = [dev(lw.router), gate, up, dev(lw.down), buf]
    L = ops.make_layer(lw.H, lw.E, lw.k, lw.F, keep[0], keep[1], keep[2], keep[3], (t, t, Q4_K),
                       n_slots=(lw.n_slots,) * 3)
    for T in (1, 3):
        x = np.random.default_rng(T + off).standard_normal((T, 2048)).astype(np.float32)
        out, xn, ids, w = ops.ffn_layer(L, dev(x), rms_eps=1e-6)
        r = orc.moe_layer(lw, x, rms_eps=1e-6)
        assert np.array_equal(host(ids), r["ids"]), f"T={T}"
        assert np.array_equal(bits(host(out)), bits(r["out"])), f"T={T}"
    assert_status_clean()


def test_stack_free_running(orc):
    """4 layers deep with RMSNorm between them, no teacher forcing: every
    layer's ids and the final output stay bit-identical."""
    note("4-layer free-running stack")
    layers = [LayerWeights(1024, 16, 4, 512, Q4_K, Q4_K, Q4_K, seed=200 + i, oracle=orc) for i in range(4)]
    gl = [_layer_gpu(lw) for lw in layers]
    x = np.random.default_rng(0).standard_normal((1, 1024)).astype(np.float32)
    xg = dev(x)
    for i, lw in enumerate(layers):
        r = orc.moe_layer(lw, x, rms_eps=1e-6)
        out, xn, ids, _ = ops.ffn_layer(gl[i][0], xg, rms_eps=1e-6)
        assert np.array_equal(host(ids), r["ids"]), f"layer {i}"
        assert np.array_equal(bits(host(xn)), bits(r["xnext"])), f"layer {i}"
        x, xg = r["xnext"], xn
