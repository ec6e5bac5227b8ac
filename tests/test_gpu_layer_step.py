"""GPU parity of the step either side of the expert FFN, through the C ABI:
the router input of a decoder layer (qwmoe_rms_norm_mul) and the shared-expert
branch of build_moe (qwmoe_shared_expert_add), alone and chained with the MoE
layer into one decoder layer's FFN half:

    ffn_in = rms_norm(h) * ffn_norm_w          (core/runtime.cpp:2028-2030)
    moe    = experts(ffn_in)                   (build_moe, 861-959)
    out    = moe + shared(ffn_in) + h          (963-972, then the residual add)

Bit for bit against the CPU oracle, which tests/test_oracle.py pins bit for bit
to the reference ggml graph of the same ops.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from questwend_amd import ops  # noqa: E402
from oracle_lib import Q4_K, Q6_K, Q8_0, LayerWeights, Oracle, SharedWeights  # noqa: E402

DEV = "cuda:0"


def note(msg: str) -> None:
    print(f"[gpu-layer-step] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.int32)


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    prev = ops.set_mfma_form(ops.MFMA_EXACT)   # bit-exact tests: the matrix cores (T = 17) replay ggml's float steps
    yield
    torch.cuda.synchronize()
    ops.set_mfma_form(prev)


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def status_clean():
    st = ops.device_status(clear=True)
    assert st & (qa.STATUS_BAD_ID | qa.STATUS_BAD_SLOT) == 0, f"device status {st}"


def gpu_shared(se: SharedWeights):
    keep = [dev(se.gate.reshape(se.F, -1)), dev(se.up.reshape(se.F, -1)), dev(se.down.reshape(se.H, -1)),
            dev(se.gate_inp)]
    return ops.make_shared_expert(se.F, *keep, (se.type_gate, se.type_up, se.type_down)), keep


@pytest.mark.parametrize("n,rows", [(2048, 1), (2048, 5), (4096, 3)])
def test_router_input_norm(orc, n, rows):
    note(f"rms_norm * weight n={n} rows={rows}")
    rng = np.random.default_rng(n + rows)
    x = (rng.standard_normal((rows, n)) * 2).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    got = host(ops.rms_norm(dev(x), 1e-6, weight=dev(w)))
    assert np.array_equal(bits(got), bits(orc.rms_norm_mul(x, w, 1e-6)))


@pytest.mark.parametrize("types", [(Q4_K, Q4_K, Q4_K), (Q4_K, Q4_K, Q6_K), (Q8_0, Q8_0, Q8_0), (Q6_K, Q6_K, Q8_0)])
@pytest.mark.parametrize("T", [1, 3, 17])
def test_shared_expert_add(orc, types, T):
    """T = 17 puts 17 rows in the one bin: the matrix cores take the
    projections (min rows 8); smaller batches stay on the GEMV.  Bit for bit
    under the exact matrix-core form; the default form at T = 17 within 1e-5."""
    note(f"shared expert types={types} T={T} (H=2048, F_sh=512)")
    se = SharedWeights(2048, 512, *types, seed=70 + T, oracle=orc)
    g, keep = gpu_shared(se)
    rng = np.random.default_rng(T + 5)
    x = rng.standard_normal((T, 2048)).astype(np.float32)
    mo = rng.standard_normal((T, 2048)).astype(np.float32)
    res = rng.standard_normal((T, 2048)).astype(np.float32)
    prev = ops.set_mfma_min_rows(8)
    try:
        for resid in (None, res):
            got = host(ops.shared_expert_add(g, dev(x), dev(mo), None if resid is None else dev(resid)))
            want = orc.shared_expert_add(se, x, mo, resid)
            assert np.array_equal(bits(got), bits(want)), f"resid={resid is not None}"
        # in place: out is moe_out
        mo_d = dev(mo)
        ops.shared_expert_add(g, dev(x), mo_d, out=mo_d)
        assert np.array_equal(bits(host(mo_d)), bits(orc.shared_expert_add(se, x, mo)))
        if T == 17:
            # the default form: gate/up exact, the down projection's matrix cores on
            # block sums (same integers, another fp32 order): within 1e-5 of max|out|
            prev_f = ops.set_mfma_form(ops.MFMA_AUTO)
            try:
                got = host(ops.shared_expert_add(g, dev(x), dev(mo)))
            finally:
                ops.set_mfma_form(prev_f)
            want = orc.shared_expert_add(se, x, mo).astype(np.float64)
            assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    finally:
        ops.set_mfma_min_rows(prev)
    status_clean()


@pytest.mark.parametrize("T", [1, 5])
def test_decoder_ffn_half(orc, T):
    """One decoder layer's FFN half at the 30B MoE shape (E=16 experts for the
    oracle's sake) with a 512-wide shared expert: router-input norm with its
    weight, the MoE layer, the shared expert and the residual add, chained on
    the GPU as a runtime would call them, against the same chain on the CPU."""
    note(f"decoder FFN half T={T}: norm*w -> MoE (E=16, k=8, F=768) -> shared (F_sh=512) + residual")
    lw = LayerWeights(2048, 16, 8, 768, Q4_K, Q4_K, Q6_K, seed=90 + T, oracle=orc)
    se = SharedWeights(2048, 512, Q4_K, Q4_K, Q6_K, seed=95 + T, oracle=orc)
    rng = np.random.default_rng(300 + T)
    h = (rng.standard_normal((T, 2048)) * 2).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    tensors = [dev(lw.router), dev(lw.gate), dev(lw.up), dev(lw.down)]
    L = ops.make_layer(lw.H, lw.E, lw.k, lw.F, *tensors, (lw.type_gate, lw.type_up, lw.type_down),
                       n_slots=(lw.n_slots,) * 3)
    g, keep = gpu_shared(se)
    hd = dev(h)
    ffn_in = ops.rms_norm(hd, 1e-6, weight=dev(nw))
    moe, _, ids, w = ops.ffn_layer(L, ffn_in)
    out = ops.shared_expert_add(g, ffn_in, moe, hd)
    # the same chain on the CPU
    x = orc.rms_norm_mul(h, nw, 1e-6)
    r = orc.moe_layer(lw, x)
    want = orc.shared_expert_add(se, x, r["out"], h)
    assert np.array_equal(host(ids), r["ids"])
    assert np.array_equal(bits(host(w)), bits(r["weights"]))
    assert np.array_equal(bits(host(out)), bits(want))
    status_clean()
