"""GPU parity of the grouped prefill path: mul_mat_id over many routed rows.

Experts with at least ``mfma_min_rows`` routed rows go to the int8 matrix-core
kernel (v_mfma_i32_16x16x64_i8), lighter ones to the bit-exact GEMV.  The bar:
router ids and the per-expert grouping exact (test_gpu_parity.py covers them at
T up to 1024), the integer block sums exact, and fp32 outputs within 1e-3 of
the CPU reference, measured as max|gpu - cpu| / max(max|cpu|, 1e-30).

The matrix cores have two forms of the float tail (qwmoe_set_mfma_form):
  * exact: ggml's eight AVX2 lane sums and four min lanes per super-block,
    formed exactly and replayed in ggml's float order -- outputs bit-identical
    to the reference;
  * block-sum: each super-block's exact integer sums scaled and added in one
    fp32 chain per output -- the same products summed in another order, within
    BS_TOL of the reference per projection.
The default is the exact form.  The opt-in auto form takes the exact form
wherever an output may be re-quantized (mul_mat_id, gate/up of a layer) and
block sums for the layers' down projections, so layer outputs stay within
BS_TOL too.  Block sums everywhere
are reported beside it: there a last-bit change of gate/up can move a
re-quantized Q8_K value by one step.  Both forms are pinned on inputs for which
every fp32 operation is exact (block scales d = dmin = 1, activations that
quantize to themselves with d = -1, sums below 2^24): there the forms and the
reference agree bit for bit.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from questwend_amd import ops  # noqa: E402
from oracle_lib import (Q4_K, Q6_K, REF_SO_AVX512, LayerWeights, Oracle, RefGGML, have_ref,  # noqa: E402
                        have_ref_avx512, row_size)

DEV = "cuda:0"
TOL = 1e-3
BS_TOL = 1e-5   # block-sum projections vs the reference, relative to max|out|
EXACT, BLOCK_SUM, AUTO = ops.MFMA_EXACT, ops.MFMA_BLOCK_SUM, ops.MFMA_AUTO


def note(msg: str) -> None:
    print(f"[gpu-prefill] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    prev = ops.set_mfma_min_rows(8)
    yield
    torch.cuda.synchronize()
    ops.set_mfma_min_rows(prev)


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def rel_err(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def encode_q4k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """The 12 scale bytes of a Q4_K block from 8 six-bit scales and mins: the
    inverse of get_scale_min_k4 (ggml-quants.c:880-887)."""
    out = np.zeros(sc.shape[:-1] + (12,), np.uint8)
    for j in range(4):
        out[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        out[..., j + 4] = (mn[..., j] & 63) | ((mn[..., j + 4] >> 4) << 6)
        out[..., j + 8] = (sc[..., j + 4] & 15) | ((mn[..., j + 4] & 15) << 4)
    return out


def exact_q4k(rng, rows: int, K: int, max_scale: int) -> np.ndarray:
    """Q4_K rows with d = dmin = 1.0 and small scales: dequantized weights are
    small integers, so every fp32 operation of the block dot is exact."""
    nb = K // 256
    blk = np.zeros((rows, nb, 144), np.uint8)
    blk[..., 0:4] = np.array([0x00, 0x3C, 0x00, 0x3C], np.uint8)   # fp16 1.0, 1.0
    sc = rng.integers(0, max_scale + 1, (rows, nb, 8)).astype(np.uint8)
    mn = rng.integers(0, 64, (rows, nb, 8)).astype(np.uint8)
    blk[..., 4:16] = encode_q4k_scales(sc, mn)
    blk[..., 16:] = rng.integers(0, 256, (rows, nb, 128)).astype(np.uint8)
    return blk.reshape(-1)


def exact_acts(rng, shape, K: int) -> np.ndarray:
    """f32 activations that Q8_K quantizes to themselves (negated, d = -1): small
    integers with one 127 per 256-block as the unique largest magnitude."""
    x = rng.integers(-31, 32, shape + (K,)).astype(np.float32)
    x[..., ::256] = 127.0
    return x


def exact_q6k(rng, rows: int, K: int, max_scale: int) -> np.ndarray:
    """Q6_K rows with d = 1.0 and scales in [-max_scale, max_scale]: dequantized
    weights sc * (q6 - 32) are small integers, every fp32 operation exact."""
    nb = K // 256
    blk = np.zeros((rows, nb, 210), np.uint8)
    blk[..., 0:192] = rng.integers(0, 256, (rows, nb, 192)).astype(np.uint8)       # ql, qh
    blk[..., 192:208] = rng.integers(-max_scale, max_scale + 1, (rows, nb, 16)).astype(np.int8).view(np.uint8)
    blk[..., 208:210] = np.array([0x00, 0x3C], np.uint8)                            # fp16 1.0
    return blk.reshape(-1)


def zipf_ids(rng, T: int, k: int, n_as: int, s: float = 1.1) -> np.ndarray:
    p = np.arange(1, n_as + 1, dtype=np.float64) ** -s
    p /= p.sum()
    return np.stack([rng.choice(n_as, k, replace=False, p=p) for _ in range(T)]).astype(np.int32)


def test_exact_inputs_pin_the_crafted_blocks(orc):
    """The crafted blocks dequantize to d*sc*q - dmin*m with d = dmin = 1 (the
    oracle's dequantizer, itself pinned against ggml), i.e. small integers."""
    rng = np.random.default_rng(0)
    w = exact_q4k(rng, 4, 512, max_scale=7)
    deq = orc.dequantize(Q4_K, w, 4 * 512)
    assert np.all(deq == np.round(deq)) and np.max(np.abs(deq)) <= 7 * 15 + 63


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("K,N,ne11,min_rows", [(2048, 128, 1, 16), (768, 256, 2, 1), (4096, 64, 1, 8)])
def test_mfma_integer_core_bit_exact(orc, K, N, ne11, min_rows, exact):
    note(f"matrix-core mul_mat_id, exact inputs: K={K} N={N} ne11={ne11} min_rows={min_rows} exact form={exact}")
    rng = np.random.default_rng(K + N)
    n_as, T, n_ids = 5, 70, 2
    w = exact_q4k(rng, n_as * N, K, max_scale=7)
    b = exact_acts(rng, (T, ne11), K)
    ids = np.stack([[0, 1 + (t % 4)] for t in range(T)]).astype(np.int32)   # expert 0 takes all 70 tokens
    want = orc.mul_mat_id(Q4_K, K, N, n_as, w, b, ids)
    prev, prev_f = ops.set_mfma_min_rows(min_rows), ops.set_mfma_form(EXACT if exact else BLOCK_SUM)
    try:
        got = host(ops.mul_mat_id(Q4_K, dev(w), K, N, n_as, dev(b), dev(ids)))
    finally:
        ops.set_mfma_min_rows(prev)
        ops.set_mfma_form(prev_f)
    assert np.array_equal(bits(got), bits(want))
    assert ops.device_status(clear=True) == 0


def full_range_q4k(rng, rows: int, K: int) -> np.ndarray:
    """Q4_K rows of random bytes (every 6-bit scale and min, every nibble) with
    positive fp16 d and dmin; row 0 at the maxima (scales, mins and nibbles 15)."""
    nb = K // 256
    blk = rng.integers(0, 256, (rows, nb, 144)).astype(np.uint8)
    blk[..., 0:2] = np.float16(rng.uniform(2.0 ** -10, 2.0 ** -6, (rows, nb))).view(np.uint8).reshape(rows, nb, 2)
    blk[..., 2:4] = np.float16(rng.uniform(2.0 ** -12, 2.0 ** -8, (rows, nb))).view(np.uint8).reshape(rows, nb, 2)
    blk[0, :, 4:] = 0xFF
    return blk.reshape(-1)


@pytest.mark.parametrize("kernel", ["f16p", "f16", "int8"])
@pytest.mark.parametrize("K,N,ne11,min_rows", [(2048, 128, 1, 1), (768, 256, 2, 8), (4096, 64, 1, 16)])
def test_mfma_exact_full_range_bit_exact(orc, K, N, ne11, min_rows, kernel, monkeypatch):
    """The exact Q4_K form on each matrix-core kernel -- the persistent f16 one
    (the default: 32-row items, two 16-row tiles per weight operand), the f16 one
    with a workgroup per (16-row item, tile) (QWMOE_MFMA_PERSIST=0; both: one
    v_mfma_f32_16x16x32_f16 per AVX lane on sc * q4 and an f16 copy of the Q8_K
    quants) or, with QWMOE_MFMA_F16=0, the int8 one -- over blocks of random bytes
    and activations whose Q8_K rows reach -128 and 127: bit-identical to ggml's
    AVX2 order (the oracle).  Expert 0 holds 70 tokens (items of 32 rows: 32, 32,
    6, the last with one tile; items of 16: a partial last one), experts 1-4 17
    or 18 (a second tile of one or two rows)."""
    note(f"exact Q4_K matrix cores, full-range blocks: kernel={kernel} K={K} N={N} ne11={ne11} min_rows={min_rows}")
    monkeypatch.setenv("QWMOE_MFMA_F16", "0" if kernel == "int8" else "1")
    monkeypatch.setenv("QWMOE_MFMA_PERSIST", "1" if kernel == "f16p" else "0")
    rng = np.random.default_rng(3 * K + N)
    n_as, T = 5, 70
    w = full_range_q4k(rng, n_as * N, K)
    b = (rng.standard_normal((T, ne11, K)) * 2.0).astype(np.float32)
    b[:, :, 7::256] = 40.0                                   # the block maximum: q8 -128 there
    b[0, :, :] = np.where(np.arange(K) % 2 == 0, 1.0, -1.0)  # every q8 -128 or 127
    ids = np.stack([[0, 1 + (t % 4)] for t in range(T)]).astype(np.int32)
    want = orc.mul_mat_id(Q4_K, K, N, n_as, w, b, ids)
    prev, prev_f = ops.set_mfma_min_rows(min_rows), ops.set_mfma_form(EXACT)
    try:
        got = host(ops.mul_mat_id(Q4_K, dev(w), K, N, n_as, dev(b), dev(ids)))
    finally:
        ops.set_mfma_min_rows(prev)
        ops.set_mfma_form(prev_f)
    assert np.array_equal(bits(got), bits(want))
    assert ops.device_status(clear=True) == 0


@pytest.mark.parametrize("K,N,T,k,n_as,ne11", [(2048, 768, 256, 8, 32, 1), (768, 2048, 128, 8, 16, 8),
                                              (2048, 512, 97, 4, 8, 1)])
def test_mfma_random(orc, K, N, T, k, n_as, ne11):
    """Random Q4_K weights and N(0,1) activations: the default (exact) form
    bit-identical to the reference, the block-sum form within BS_TOL of it."""
    note(f"matrix-core mul_mat_id, random data: K={K} N={N} T={T} k={k} n_as={n_as} ne11={ne11}")
    rng = np.random.default_rng(T + N)
    w = orc.quantize(Q4_K, (rng.standard_normal((n_as * N, K)) * 0.02).astype(np.float32))
    b = rng.standard_normal((T, ne11, K)).astype(np.float32)
    ids = zipf_ids(rng, T, k, n_as)
    want = orc.mul_mat_id(Q4_K, K, N, n_as, w, b, ids)
    counts = np.bincount(ids.reshape(-1), minlength=n_as)
    assert counts.max() >= 32, "the case must route some expert to the matrix cores"
    wd, bd, idd = dev(w), dev(b), dev(ids)
    got_auto = host(ops.mul_mat_id(Q4_K, wd, K, N, n_as, bd, idd))
    prev = ops.set_mfma_form(BLOCK_SUM)
    try:
        got = host(ops.mul_mat_id(Q4_K, wd, K, N, n_as, bd, idd))
    finally:
        ops.set_mfma_form(prev)
    note(f"  heavy experts {int((counts >= 32).sum())}/{n_as}, max rows {counts.max()}, "
         f"block-sum rel err {rel_err(got, want):.3e}")
    assert prev == EXACT   # the library's default
    assert np.array_equal(bits(got_auto), bits(want))
    assert rel_err(got, want) < BS_TOL
    assert ops.device_status(clear=True) == 0


def test_exact_inputs_pin_the_crafted_q6k_blocks(orc):
    """The crafted Q6_K blocks dequantize to sc * (q6 - 32) with d = 1 (the
    oracle's dequantizer, pinned against ggml), i.e. small integers."""
    rng = np.random.default_rng(1)
    w = exact_q6k(rng, 4, 512, max_scale=4)
    deq = orc.dequantize(Q6_K, w, 4 * 512)
    assert np.all(deq == np.round(deq)) and np.max(np.abs(deq)) <= 4 * 32


@pytest.mark.parametrize("form", ["block_sum", "exact"])
@pytest.mark.parametrize("K,N,min_rows", [(768, 128, 8), (1536, 64, 1), (512, 192, 16)])
def test_mfma_q6k_integer_core_bit_exact(orc, K, N, min_rows, form):
    """Q6_K heavy experts on the matrix cores (K = 768 puts every other
    super-block 2 bytes past a dword boundary in odd rows) on exact inputs:
    bit-identical to the reference in both forms (the exact form's base-64
    digits of sc * q6 and its bsum term included: scales span [-128, 127])."""
    note(f"Q6_K matrix-core mul_mat_id ({form} form), exact inputs: K={K} N={N} min_rows={min_rows}")
    rng = np.random.default_rng(K + N + 6)
    n_as, T = 5, 70
    w = exact_q6k(rng, n_as * N, K, max_scale=4)
    if form == "exact":   # the extreme scales and 6-bit values: the digits' range ends
        wb = w.reshape(n_as * N, K // 256, 210)
        wb[:, :, 192:208] = rng.choice(np.array([-128, -127, -1, 0, 1, 126, 127], np.int8),
                                       wb[:, :, 192:208].shape).view(np.uint8)
        wb[0, :, 0:192] = 0xFF                    # row 0: every q6 = 63
    b = exact_acts(rng, (T, 1), K)
    ids = np.stack([[0, 1 + (t % 4)] for t in range(T)]).astype(np.int32)   # expert 0 takes all 70 tokens
    want = orc.mul_mat_id(Q6_K, K, N, n_as, w, b, ids)
    prev, prev_f = ops.set_mfma_min_rows(min_rows), ops.set_mfma_form(BLOCK_SUM if form == "block_sum" else EXACT)
    try:
        got = host(ops.mul_mat_id(Q6_K, dev(w), K, N, n_as, dev(b), dev(ids)))
    finally:
        ops.set_mfma_min_rows(prev)
        ops.set_mfma_form(prev_f)
    assert np.array_equal(bits(got), bits(want))
    assert ops.device_status(clear=True) == 0


@pytest.mark.parametrize("K,N,T,k,n_as", [(1536, 256, 256, 8, 16), (768, 2048, 128, 8, 16), (512, 64, 97, 4, 8)])
def test_mfma_q6k_random(orc, K, N, T, k, n_as):
    """Random Q6_K weights and N(0,1) activations: block sums within BS_TOL of the
    reference; the default form (exact for mul_mat_id, so Q6_K stays on the
    GEMV) bit-identical."""
    note(f"Q6_K matrix-core mul_mat_id, random data: K={K} N={N} T={T} k={k} n_as={n_as}")
    rng = np.random.default_rng(T + N + 6)
    w = orc.quantize(Q6_K, (rng.standard_normal((n_as * N, K)) * 0.02).astype(np.float32))
    b = rng.standard_normal((T, 1, K)).astype(np.float32)
    ids = zipf_ids(rng, T, k, n_as)
    want = orc.mul_mat_id(Q6_K, K, N, n_as, w, b, ids)
    counts = np.bincount(ids.reshape(-1), minlength=n_as)
    assert counts.max() >= 32, "the case must route some expert to the matrix cores"
    wd, bd, idd = dev(w), dev(b), dev(ids)
    got_auto = host(ops.mul_mat_id(Q6_K, wd, K, N, n_as, bd, idd))
    prev = ops.set_mfma_form(BLOCK_SUM)
    try:
        got = host(ops.mul_mat_id(Q6_K, wd, K, N, n_as, bd, idd))
    finally:
        ops.set_mfma_form(prev)
    note(f"  heavy experts {int((counts >= 8).sum())}/{n_as}, max rows {counts.max()}, "
         f"block-sum rel err {rel_err(got, want):.3e}")
    assert np.array_equal(bits(got_auto), bits(want))
    assert rel_err(got, want) < BS_TOL
    assert ops.device_status(clear=True) == 0


def test_mfma_disabled_is_bit_exact(orc):
    note("mul_mat_id with the matrix cores disabled: every expert on the GEMV, bit-exact")
    rng = np.random.default_rng(11)
    K, N, T, k, n_as = 2048, 256, 96, 4, 8
    w = orc.quantize(Q4_K, (rng.standard_normal((n_as * N, K)) * 0.02).astype(np.float32))
    b = rng.standard_normal((T, 1, K)).astype(np.float32)
    ids = zipf_ids(rng, T, k, n_as)
    prev = ops.set_mfma_min_rows(0)
    try:
        got = host(ops.mul_mat_id(Q4_K, dev(w), K, N, n_as, dev(b), dev(ids)))
    finally:
        ops.set_mfma_min_rows(prev)
    assert np.array_equal(bits(got), bits(orc.mul_mat_id(Q4_K, K, N, n_as, w, b, ids)))


def layer_forms(layer, x):
    """ffn_layer under the exact form (the default; all four outputs), the
    opt-in auto form and block sums everywhere (outputs only)."""
    prev = ops.set_mfma_form(EXACT)
    try:
        out, xn, ids, w = (host(t) for t in ops.ffn_layer(layer, dev(x), rms_eps=1e-6))
        ops.set_mfma_form(AUTO)
        out_auto = host(ops.ffn_layer(layer, dev(x), rms_eps=1e-6)[0])
        ops.set_mfma_form(BLOCK_SUM)
        out_bs = host(ops.ffn_layer(layer, dev(x), rms_eps=1e-6)[0])
    finally:
        ops.set_mfma_form(prev)
    return out, xn, ids, w, out_auto, out_bs


class GpuLayerQ4K:
    """A Q4_K layer generated and quantized on the GPU, with a host copy for the
    CPU reference.  Router rows scaled by a Zipf profile skew expert popularity."""

    def __init__(self, H, E, k, F, seed, zipf_skew=1.1):
        from oracle_lib import zipf_row_scales
        self.router = torch.empty((E, H), dtype=torch.float32, device=DEV)
        ops.randn_(self.router, seed * 10 + 1, 0.0, 0.02)
        self.router *= dev(zipf_row_scales(E, zipf_skew))[:, None]
        mats = []
        tmp = torch.empty(E * F * H, dtype=torch.float32, device=DEV)
        for j, (rows, cols) in enumerate(((F, H), (F, H), (H, F))):
            ops.randn_(tmp, seed * 10 + 2 + j, 0.0, 0.02)
            mats.append(ops.quantize_chunk(Q4_K, tmp.view(E * rows, cols)).view(E, -1))
        del tmp
        self.gate, self.up, self.down = mats
        self.layer = ops.make_layer(H, E, k, F, self.router, self.gate, self.up, self.down, (Q4_K,) * 3)
        torch.cuda.synchronize()
        lw = LayerWeights.__new__(LayerWeights)
        lw.H, lw.E, lw.k, lw.F = H, E, k, F
        lw.type_gate = lw.type_up = lw.type_down = Q4_K
        lw.router = self.router.cpu().numpy()
        lw.gate, lw.up, lw.down = (m.cpu().numpy().reshape(-1) for m in mats)
        lw.n_slots, lw.slot_of = E, None
        self.host = lw


@pytest.mark.parametrize("T", [512])
def test_prefill_layer_30b_shape(orc, T):
    """a Q4_K layer at the 30B-A3B shape, T tokens of N(0,1), Zipf-skewed
    routing: ids and weights bit-identical to the CPU reference; the layer output
    bit-identical with the exact matrix-core form and within BS_TOL with the
    auto form; its RMSNorm within 1e-3 (double sum in another order,
    rounding identical except within ~2^-29 of a float boundary).

    With block sums everywhere the gate/up outputs can differ in the last bit,
    and the layer re-quantizes SwiGLU(gate, up) to Q8_K before the down
    projection: a value at a rounding boundary moves by one int8 step, which
    moves the token's output by d_q8 * w.  That gap is reported (the
    reference's own AVX-512 build beside it) and only bounded loosely here."""
    H, E, k, F = 2048, 128, 8, 768
    note(f"prefill layer 30B shape T={T} (reference: {'ggml' if have_ref() else 'oracle'})")
    g = GpuLayerQ4K(H, E, k, F, seed=77)
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, H)).astype(np.float32)
    out, xn, ids, w, out_auto, out_bs = layer_forms(g.layer, x)
    if have_ref():
        r = RefGGML().layer(g.host, T, rms_eps=1e-6, n_threads=16)(x)
    else:
        r = orc.moe_layer(g.host, x, rms_eps=1e-6)
    counts = np.bincount(r["ids"].reshape(-1), minlength=E)
    note(f"  rows per expert: max {counts.max()}, experts >= 32 rows: {int((counts >= 32).sum())}, "
         f"unused: {int((counts == 0).sum())}")
    # the configured skew: counts from 0 to a few hundred, Zipf-like in between
    from bench import row_count_profile
    prof = row_count_profile(counts)
    assert prof["max_rows"] >= 150 and prof["experts_with_no_rows"] >= 1, prof
    assert -1.6 < prof["loglog_slope_rank5_100"] < -0.7, prof
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(bits(w), bits(r["weights"]))
    note(f"  output rel err: exact {rel_err(out, r['out']):.3e}, auto {rel_err(out_auto, r['out']):.3e}, "
         f"block sums everywhere {rel_err(out_bs, r['out']):.3e}; rms_norm {rel_err(xn, r['xnext']):.3e}")
    if have_ref() and have_ref_avx512():
        o5 = RefGGML(REF_SO_AVX512).layer(g.host, T, rms_eps=1e-6, n_threads=16)(x)["out"]
        note(f"  reference AVX-512 build vs AVX2 build: rel err {rel_err(o5, r['out']):.3e}")
    assert np.array_equal(bits(out), bits(r["out"]))
    assert rel_err(out_auto, r["out"]) < BS_TOL
    assert rel_err(out_bs, r["out"]) < 1e-2
    assert rel_err(xn, r["xnext"]) < TOL


class GpuLayerTyped:
    """A layer of any weight types generated and quantized on the GPU, with a host
    copy for the CPU reference.  Optional Zipf-scaled router rows skew expert
    popularity; optional permuted slot pools (logical expert e lives in slot p[e])."""

    def __init__(self, H, E, k, F, types, seed, zipf_skew=None, permute=False):
        from oracle_lib import zipf_row_scales
        tg, tu, td = types
        self.router = torch.empty((E, H), dtype=torch.float32, device=DEV)
        ops.randn_(self.router, seed * 10 + 1, 0.0, 0.02)
        if zipf_skew is not None:
            self.router *= dev(zipf_row_scales(E, zipf_skew))[:, None]
        mats = []
        tmp = torch.empty(E * F * H, dtype=torch.float32, device=DEV)
        for j, (t, rows, cols) in enumerate(((tg, F, H), (tu, F, H), (td, H, F))):
            ops.randn_(tmp, seed * 10 + 2 + j, 0.0, 0.02)
            mats.append(ops.quantize_chunk(t, tmp.view(E * rows, cols)).view(E, -1))
        del tmp
        slots = None
        if permute:
            g = torch.Generator().manual_seed(seed)
            perms = [torch.randperm(E, generator=g).to(torch.int32) for _ in range(3)]
            pools = []
            for m, p in zip(mats, perms):
                pool = torch.empty_like(m)
                pool[p.long().to(DEV)] = m
                pools.append(pool)
            mats = pools
            slots = tuple(p.to(DEV) for p in perms)
        self.mats, self.slots = mats, slots
        self.layer = ops.make_layer(H, E, k, F, self.router, *mats, types, n_slots=(E, E, E), slots=slots)
        torch.cuda.synchronize()
        lw = LayerWeights.__new__(LayerWeights)
        lw.H, lw.E, lw.k, lw.F = H, E, k, F
        lw.type_gate, lw.type_up, lw.type_down = types
        lw.router = self.router.cpu().numpy()
        lw.gate, lw.up, lw.down = (m.cpu().numpy().reshape(-1) for m in mats)
        lw.n_slots = E
        lw.slot_of = None if slots is None else tuple(s.cpu().numpy() for s in slots)
        self.host = lw


C5 = (4096, 128, 8, 1536, (Q4_K, Q4_K, Q6_K))   # configs[4]: large experts, Q6_K down


@pytest.mark.parametrize("T", [1, 5])
def test_layer_config5_shape_permuted_slots(orc, T):
    """configs[4] shape (H=4096, F=1536, Q4_K gate/up, Q6_K down, E=128) read
    through permuted slot pools: ids, weights, output and RMSNorm bit-identical
    to the oracle (whose slot handling the parity tests pin at smaller shapes)."""
    H, E, k, F, types = C5
    note(f"ffn_layer config-5 shape T={T}, permuted slots")
    ops.device_status(clear=True)
    g = GpuLayerTyped(H, E, k, F, types, seed=900 + T, permute=True)
    x = np.random.default_rng(T + 50).standard_normal((T, H)).astype(np.float32)
    out, xn, ids, w = ops.ffn_layer(g.layer, dev(x), rms_eps=1e-6)
    out, xn, ids, w = host(out), host(xn), host(ids), host(w)
    r = orc.moe_layer(g.host, x, rms_eps=1e-6)
    assert np.array_equal(ids, r["ids"])
    assert np.array_equal(bits(w), bits(r["weights"]))
    assert np.array_equal(bits(out), bits(r["out"]))
    assert np.array_equal(bits(xn), bits(r["xnext"]))
    assert ops.device_status(clear=True) == 0


def test_prefill_layer_config5_shape():
    """configs[4] prefill: T=1024 at the large-expert shape, Zipf-skewed routing.
    Q4_K gate/up of the heavy experts run on the matrix cores, the Q6_K down on
    the GEMV.  Against the reference ggml (16 threads) when it is built; else
    tokens are independent, so a sample of 24 tokens is checked against the
    oracle.  Output bit-identical with the exact matrix-core form, within
    BS_TOL with the auto form (block sums everywhere: reported, as in
    test_prefill_layer_30b_shape)."""
    H, E, k, F, types = C5
    T = 1024
    note(f"prefill layer config-5 shape T={T} (reference: {'ggml' if have_ref() else 'oracle, 24 tokens'})")
    g = GpuLayerTyped(H, E, k, F, types, seed=950, zipf_skew=1.1)
    x = np.random.default_rng(T).standard_normal((T, H)).astype(np.float32)
    out, xn, ids, w, out_auto, out_bs = layer_forms(g.layer, x)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    note(f"  rows per expert: max {counts.max()}, experts >= 8 rows: {int((counts >= 8).sum())}")
    assert counts.max() >= 64, "the case must route heavy experts to the matrix cores"
    if have_ref():
        r = RefGGML().layer(g.host, T, rms_eps=1e-6, n_threads=16)(x)
        sel = np.arange(T)
    else:
        sel = np.r_[0:8, 500:508, T - 8:T]
        r = Oracle().moe_layer(g.host, x[sel], rms_eps=1e-6)
    assert np.array_equal(ids[sel], r["ids"])
    assert np.array_equal(bits(w[sel]), bits(r["weights"]))
    assert np.array_equal(bits(out[sel]), bits(r["out"]))
    note(f"  output rel err: auto {rel_err(out_auto[sel], r['out']):.3e}, "
         f"block sums everywhere {rel_err(out_bs[sel], r['out']):.3e}")
    assert rel_err(out_auto[sel], r["out"]) < BS_TOL
    assert rel_err(out_bs[sel], r["out"]) < 1e-2
    assert rel_err(xn[sel], r["xnext"]) < TOL
    assert ops.device_status(clear=True) == 0
