"""The allocation-free mul_mat_id (qwmoe_mul_mat_id_noalloc) against
qwmoe_mul_mat_id, bit for bit, through the C ABI.

Each case makes two calls in a row on the same static scratch, the second
with a smaller input.  The first is large enough for the matrix-core kernel
to take part (Q4_K).  The second feeds b per id (ne11 = n_ids, the down
projection's layout).  An input larger than the scratch is rejected before
anything runs.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402
from questwend_amd import ops  # noqa: E402
from oracle_lib import Q4_K, Q6_K, Q8_0  # noqa: E402

DEV = "cuda:0"
QWMOE_ERR_SCRATCH = -8


def note(msg: str) -> None:
    print(f"[gpu-noalloc] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 512 << 20)
    yield
    torch.cuda.synchronize()


def weights(t: int, K: int, N: int, n_as: int, seed: int):
    x = torch.empty((n_as * N, K), dtype=torch.float32, device=DEV)
    ops.randn_(x, seed, 0.0, 0.02)
    return ops.quantize_chunk(t, x)


def inputs(K: int, n_as: int, T: int, n_ids: int, ne11: int, seed: int):
    b = torch.empty((T, ne11, K), dtype=torch.float32, device=DEV)
    ops.randn_(b, seed, 0.0, 1.0)
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(n_as, n_ids, replace=False) for _ in range(T)]).astype(np.int32)
    return b, torch.from_numpy(ids).to(DEV)


@pytest.mark.parametrize("t,K,N", [(Q4_K, 2048, 768), (Q6_K, 768, 2048), (Q8_0, 2048, 256)])
def test_noalloc_equals_mul_mat_id_two_calls(t, K, N):
    n_as = 16
    w = weights(t, K, N, n_as, seed=K + N + t)
    for T, n_ids, ne11 in ((64, 8, 1), (3, 8, 8)):
        note(f"type={t} K={K} N={N} n_as={n_as} T={T} n_ids={n_ids} ne11={ne11}")
        b, ids = inputs(K, n_as, T, n_ids, ne11, seed=T + ne11)
        want = ops.mul_mat_id(t, w, K, N, n_as, b, ids)
        got = ops.mul_mat_id(t, w, K, N, n_as, b, ids, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), f"T={T}"
    st = ops.device_status(clear=True)
    assert st & (qa.STATUS_BAD_ID | qa.STATUS_BAD_SLOT) == 0, f"device status {st}"


def test_noalloc_rejects_input_beyond_scratch():
    note("noalloc: 4096 tokens x K=4096 (16 MiB of Q8_K rows) rejected before any launch")
    K, N, n_as, T = 4096, 16, 2, 4096
    w = weights(Q4_K, K, N, n_as, seed=3)
    b = torch.zeros((T, 1, K), dtype=torch.float32, device=DEV)
    ids = torch.zeros((T, 1), dtype=torch.int32, device=DEV)
    with pytest.raises(qa.QwmoeError) as e:
        ops.mul_mat_id(Q4_K, w, K, N, n_as, b, ids, noalloc=True)
    assert e.value.status == QWMOE_ERR_SCRATCH
    # the entry point with the library workspace takes the same call
    out = ops.mul_mat_id(Q4_K, w, K, N, n_as, b, ids)
    torch.cuda.synchronize()
    assert torch.equal(out, torch.zeros_like(out))
