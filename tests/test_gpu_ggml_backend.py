"""The QWMOE ggml backend (include/ggml-qwmoe.h, questwend_amd/libggml-qwmoe.so)
under ggml's own scheduler: build_moe's graph (core/runtime.cpp:861-974, with
an RMSNorm after it) runs through ggml_backend_sched with QWMOE first and the
reference CPU backend second (oracle/backend_driver.cpp).  The experts live in
a QWMOE buffer, so the scheduler hands the three mul_mat_id nodes to QWMOE and
the router, softmax, top-k, SwiGLU and weighted sum to the CPU.  Checked: all
three mul_mat_id nodes ran on QWMOE, and ids, the layer output and its RMSNorm
equal the CPU-only graph (oracle/_ref) bit for bit, for decode (T = 1), a
small batch and a batch whose heavy experts take the matrix cores, over Q4_K,
mixed Q4_K / Q6_K and Q8_0 experts."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from oracle_lib import LayerWeights, Oracle, Q4_K, Q6_K, Q8_0, RefGGML, have_ref  # noqa: E402

ROOT = Path(__file__).resolve().parents[1]
BE_SO = ROOT / "oracle" / "_ref" / "libqwbe.so"


def note(msg: str) -> None:
    print(f"[gpu-ggml-backend] {msg}", flush=True)


@pytest.fixture(scope="module")
def be():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not (have_ref() and BE_SO.exists()):
        pytest.skip("oracle/_ref/libqwbe.so (the reference ggml and the backend driver) not built")
    L = C.CDLL(str(BE_SO))
    P, I64, I = C.c_void_p, C.c_int64, C.c_int
    L.qwbe_sched_moe.argtypes = [I64] * 5 + [I] * 3 + [P] * 4 + [C.c_float] + [P] * 6 + [I]
    L.qwbe_registry.argtypes = [C.c_char_p, I]
    return L


def _p(a):
    return C.c_void_p(a.ctypes.data)


def test_registry_reports_the_gpu(be):
    name = C.create_string_buffer(64)
    n = be.qwbe_registry(name, 64)
    note(f"QWMOE registry: {n} device(s), first {name.value.decode()}")
    assert n >= 1 and name.value == b"QWMOE0"


@pytest.mark.parametrize("types,T", [((Q4_K,) * 3, 1), ((Q4_K, Q4_K, Q6_K), 3), ((Q4_K,) * 3, 48),
                                     ((Q8_0,) * 3, 2)])
def test_sched_moe_equals_cpu_graph(be, types, T):
    H, E, k, F = 1024, 32, 4, 512
    note(f"build_moe through ggml_backend_sched [QWMOE, CPU]: H={H} E={E} k={k} F={F} types={types} T={T}")
    lw = LayerWeights(H, E, k, F, *types, seed=100 + T, oracle=Oracle())
    x = np.random.default_rng(T).standard_normal((T, H)).astype(np.float32)
    want = RefGGML().layer(lw, T, rms_eps=1e-6, n_threads=8)(x)
    out = np.zeros((T, H), np.float32)
    xn = np.zeros((T, H), np.float32)
    ids = np.zeros((T, k), np.int32)
    n_splits, n_mmid = C.c_int(0), C.c_int(0)
    rc = be.qwbe_sched_moe(H, E, k, F, T, *types, _p(lw.router), _p(lw.gate), _p(lw.up), _p(lw.down), 1e-6, _p(x),
                           _p(out), _p(xn), _p(ids), C.byref(n_splits), C.byref(n_mmid), 8)
    assert rc == 0, rc
    note(f"  splits {n_splits.value}, mul_mat_id nodes on QWMOE {n_mmid.value}/3")
    assert n_mmid.value == 3 and n_splits.value >= 2
    assert np.array_equal(ids, want["ids"])
    assert np.array_equal(out.view(np.uint32), want["out"].view(np.uint32))
    assert np.array_equal(xn.view(np.uint32), want["xnext"].view(np.uint32))
