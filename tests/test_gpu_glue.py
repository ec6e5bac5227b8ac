"""The ggml backend glue (include/qwmoe_ggml.h) run on a real ggml graph's
GGML_OP_MUL_MAT_ID node: build_moe's routing (soft_max -> argsort_top_k, whose
[k, T] result is a strided view with nb[1] = n_as * 4) feeding mul_mat_id over
[K, N, n_as] expert tensors.  oracle/_ref/libqwglue.so builds the graph with
the reference's own ggml (CPU backend, from its sources), computes it, copies
the node's tensors to device memory with their ne / nb untouched and calls
qwmoe_ggml_mul_mat_id on them.  The two destinations must agree bit for bit
(matrix cores, when bins reach them, in the exact form).
"""
from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from questwend_amd import ops  # noqa: E402
from oracle_lib import Q4_K, Q6_K, Q8_0  # noqa: E402

GLUE = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libqwglue.so"


def note(msg: str) -> None:
    print(f"[gpu-glue] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not GLUE.exists():
        pytest.skip("oracle/_ref/libqwglue.so not built (needs the reference tree at build time)")
    ops.init(0, 256 << 20)
    prev = ops.set_mfma_form(ops.MFMA_EXACT)
    yield
    torch.cuda.synchronize()
    ops.set_mfma_form(prev)


@pytest.fixture(scope="module")
def glue():
    lib = C.CDLL(str(GLUE))
    lib.qwglue_mul_mat_id.restype = C.c_int
    lib.qwglue_mul_mat_id.argtypes = [C.c_int] + [C.c_int64] * 6 + [C.c_void_p] * 7
    return lib


def _p(a):
    return a.ctypes.data


@pytest.mark.parametrize("type_,K,N,n_as,ne11,T,k", [(Q4_K, 1024, 256, 16, 1, 5, 4), (Q4_K, 512, 128, 8, 4, 40, 4),
                                                    (Q6_K, 768, 192, 16, 1, 3, 8), (Q6_K, 512, 128, 8, 2, 20, 2),
                                                    (Q8_0, 256, 64, 8, 1, 33, 3), (Q8_0, 512, 128, 32, 1, 1, 8)])
def test_ggml_mul_mat_id_node_through_glue(glue, type_, K, N, n_as, ne11, T, k):
    note(f"glue: type {type_} K={K} N={N} n_as={n_as} ne11={ne11} T={T} k={k}")
    rng = np.random.default_rng(K + N + T + type_)
    w = (rng.standard_normal((n_as, N, K)) * 0.02).astype(np.float32)
    b = rng.standard_normal((T, ne11, K)).astype(np.float32)
    scores = rng.standard_normal((T, n_as)).astype(np.float32)
    ids = np.zeros((T, k), np.int32)
    cpu = np.zeros((T, k, N), np.float32)
    gpu = np.zeros((T, k, N), np.float32)
    st = C.c_int(-99)
    rc = glue.qwglue_mul_mat_id(type_, K, N, n_as, ne11, T, k, _p(w), _p(b), _p(scores), _p(ids), _p(cpu), _p(gpu),
                                C.addressof(st))
    assert rc == 0 and st.value == 0, (rc, st.value)
    assert np.array_equal(ids, np.argsort(-scores, axis=1, kind="stable")[:, :k])   # no ties in random scores
    assert np.array_equal(gpu.view(np.int32), cpu.view(np.int32))
    assert ops.device_status(clear=True) == 0
