"""CPU tests of the C-ABI library: it loads, exports every symbol the header
declares, and its host-side logic (argsort replay, slot table) is correct.
No GPU compute is called here."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import questwend_amd as qa
from oracle_lib import Oracle

HEADER = Path(__file__).resolve().parents[1] / "include" / "qwmoe.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qwmoe_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = qa.lib()
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/qwmoe.h but not exported"
    assert set(names) == set(qa.SIGNATURES), "ctypes signature table out of sync with the header"


def test_status_strings_and_row_sizes():
    lib = qa.lib()
    assert lib.qwmoe_strerror(0) == b"ok"
    assert lib.qwmoe_strerror(-4) == b"workspace too small"
    assert lib.qwmoe_row_size(qa.Q4_K, 2048) == 1152
    assert lib.qwmoe_row_size(qa.Q6_K, 1536) == 1260
    assert lib.qwmoe_row_size(qa.Q8_0, 2048) == 2176
    assert lib.qwmoe_row_size(qa.Q8_K, 768) == 876
    assert lib.qwmoe_row_size(qa.Q4_K, 100) == 0
    assert lib.qwmoe_vec_dot_type(qa.Q4_K) == qa.Q8_K
    assert lib.qwmoe_vec_dot_type(qa.Q8_0) == qa.Q8_0


def test_calls_before_init_fail_cleanly():
    lib = qa.lib()
    ids = np.zeros(8, np.int32)
    rc = lib.qwmoe_group_by_expert(None, ids.ctypes.data, 8, 1, 32, 128, None, None, ids.ctypes.data)
    assert rc == -5  # QWMOE_ERR_NOT_INITIALIZED: no device work attempted


def _sort_replay(values: np.ndarray) -> np.ndarray:
    idx = np.zeros(len(values), np.int32)
    v = np.ascontiguousarray(values, np.float32)
    assert qa.lib().qwmoe_host_argsort_desc(v.ctypes.data, len(v), idx.ctypes.data) == 0
    return idx


@pytest.mark.parametrize("n", [1, 2, 7, 16, 17, 33, 64, 128, 256, 512])
def test_argsort_replay_equals_std_sort_with_ties(n):
    """The router's tie path must reproduce libstdc++'s unstable std::sort exactly."""
    orc = Oracle()
    rng = np.random.default_rng(n)
    for trial in range(200):
        levels = int(rng.integers(1, max(2, n // 2) + 1))
        v = rng.integers(0, levels, n).astype(np.float32) / np.float32(levels)
        if trial % 3 == 0:
            v = np.sort(v)[::-1].copy()          # presorted descending
        elif trial % 3 == 1:
            v = np.sort(v).copy()                # presorted ascending
        want = orc.argsort_desc(v.reshape(1, n))[0]
        assert np.array_equal(_sort_replay(v), want), (n, trial)


def test_argsort_replay_all_equal_and_probabilities():
    orc = Oracle()
    v = np.full(128, 0.0078125, np.float32)
    assert np.array_equal(_sort_replay(v), orc.argsort_desc(v.reshape(1, -1))[0])
    rng = np.random.default_rng(0)
    p = orc.soft_max((rng.standard_normal((1, 128)) * 2).astype(np.float32))[0]
    p[[3, 40, 77]] = p.max()                     # a three-way tie at the top
    assert np.array_equal(_sort_replay(p), orc.argsort_desc(p.reshape(1, -1))[0])


def test_slot_table_semantics():
    lib = qa.lib()
    t = lib.qwmoe_slot_table_create(4, 8)
    assert t
    try:
        assert lib.qwmoe_slot_table_slot_of(t, 0, 0, 0) == -1          # unassigned is -1, never 0
        assert lib.qwmoe_slot_table_fill(t, 0) == 0
        assert lib.qwmoe_slot_table_slot_of(t, 2, 3, 5) == 3 * 8 + 5    # identity: key = layer * E + expert
        assert lib.qwmoe_slot_table_fill(t, 1234) == 0
        for role in range(3):
            seen = []
            for layer in range(4):
                row = C.cast(lib.qwmoe_slot_table_row(t, role, layer), C.POINTER(C.c_int32))
                seen += [row[e] for e in range(8)]
                assert [lib.qwmoe_slot_table_slot_of(t, role, layer, e) for e in range(8)] == \
                    [row[e] for e in range(8)]
            assert sorted(seen) == list(range(32))                       # a permutation of the pool
        assert lib.qwmoe_slot_table_set(t, 1, 2, 3, 7) == 0
        assert lib.qwmoe_slot_table_slot_of(t, 1, 2, 3) == 7
        assert lib.qwmoe_slot_table_set(t, 3, 0, 0, 0) == -1
        assert lib.qwmoe_slot_table_set(t, 0, 4, 0, 0) == -1
    finally:
        lib.qwmoe_slot_table_free(t)


@pytest.mark.skipif(not Path("/root/reference/third_party/ggml/include/ggml.h").exists(),
                    reason="ggml headers (reference tree) absent")
@pytest.mark.parametrize("lang", ["c", "c++"])
def test_ggml_glue_header_compiles(tmp_path, lang):
    """include/qwmoe_ggml.h, included after ggml.h, compiles as C and as C++."""
    import shutil
    import subprocess
    cc = shutil.which("gcc" if lang == "c" else "g++")
    if cc is None:
        pytest.skip("no host compiler")
    src = tmp_path / ("glue.c" if lang == "c" else "glue.cpp")
    src.write_text('#include "ggml.h"\n#include "qwmoe_ggml.h"\n'
                   "int probe(const struct ggml_tensor * t) { return qwmoe_ggml_supports_mul_mat_id(t); }\n")
    root = Path(__file__).resolve().parents[1]
    subprocess.run([cc, "-fsyntax-only", "-Wall", "-Werror", "-x", lang, "-I", "/root/reference/third_party/ggml/include",
                    "-I", str(root / "include"), str(src)], check=True)


GGML_HEADER = Path(__file__).resolve().parents[1] / "include" / "ggml-qwmoe.h"
GGML_PLUGIN = Path(__file__).resolve().parents[1] / "questwend_amd" / "libggml-qwmoe.so"


def test_ggml_backend_plugin_exports_its_header():
    """The ggml backend plugin exports what include/ggml-qwmoe.h declares and
    leaves only ggml's own API to the host process (no GPU needed: the registry
    reports the devices HIP sees, none here)."""
    if not GGML_PLUGIN.exists():
        pytest.skip("libggml-qwmoe.so is built only where the ggml headers are present")
    text = re.sub(r"/\*.*?\*/", "", GGML_HEADER.read_text(), flags=re.S)
    names = sorted(set(re.findall(r"\b(ggml_backend_(?:qwmoe|is_qwmoe)[a-z0-9_]*)\s*\(", text)))
    assert names == ["ggml_backend_is_qwmoe", "ggml_backend_qwmoe_init", "ggml_backend_qwmoe_reg"]
    qa.lib()
    from oracle_lib import REF_SO, have_ref
    if not have_ref():
        pytest.skip("the plugin resolves ggml's symbols from a loaded ggml (oracle/_ref)")
    # In a child process: a ggml loaded RTLD_GLOBAL here would interpose its
    # symbols on every ggml build the later tests load (the AVX-512 one).
    code = ("import ctypes as C, sys\n"
            f"C.CDLL({str(REF_SO)!r}, mode=C.RTLD_GLOBAL)\n"
            f"p = C.CDLL({str(GGML_PLUGIN)!r})\n"
            f"sys.exit(0 if all(hasattr(p, n) for n in {names!r}) else 3)\n")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
