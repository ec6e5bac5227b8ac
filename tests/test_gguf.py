"""CPU tests of the GGUF reader (qwmoe_gguf_*): no GPU needed.

Fixtures are regenerated here with tests/gguf_writer.py and must hash to the
values tests/golden/gen_gguf.py recorded after checking them byte for byte
against the reference ggml's own gguf writer.  The library's view of every file
-- shards, KV pairs with their types and values, tensor infos -- must equal the
reference reader's recorded view, and the library must reject exactly the
malformed variants the reference reader rejects.
"""
from __future__ import annotations

import struct

import pytest

import questwend_amd as qa
from questwend_amd import ops
import gguf_fixtures as FX
from oracle_lib import Oracle

QWMOE_ERR_FORMAT, QWMOE_ERR_IO, QWMOE_ERR_INVALID_ARG = -6, -7, -1


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    d = tmp_path_factory.mktemp("gguf")
    hashes = FX.write_all(d, Oracle())
    return d, hashes


def test_fixtures_regenerate_byte_identical(files):
    """The regenerated files are the ones the reference writer produced."""
    _, hashes = files
    gold = FX.golden()["files"]
    assert set(hashes) == set(gold)
    for name, h in hashes.items():
        assert h == gold[name]["sha256"], name


def _norm(v):
    return [float(x) if isinstance(x, float) else x for x in v] if isinstance(v, list) else v


@pytest.mark.parametrize("name", ["moe_tiny.gguf", "moe_tiny_a64.gguf"])
def test_metadata_equals_reference_reader(files, name):
    d, _ = files
    ref = FX.golden()["files"][name]
    with ops.Gguf(d / name) as g:
        (sh,) = g.shards()
        assert (sh["version"], sh["alignment"], sh["data_offset"]) == (ref["version"], ref["alignment"],
                                                                       ref["data_offset"])
        kv = g.kv()
        assert [e["key"] for e in kv] == [e["key"] for e in ref["kv"]]
        for mine, r in zip(kv, ref["kv"]):
            assert mine["type"] == r["type"], r["key"]
            if r["type"] == 9:
                assert (mine["arr_type"], mine["n"]) == (r["arr_type"], r["n"]), r["key"]
            assert _norm(mine["value"]) == _norm(r["value"]), r["key"]
        ts = g.tensors()
        assert len(ts) == len(ref["tensors"])
        for mine, r in zip(ts, ref["tensors"]):
            assert (mine["name"], mine["type"], mine["ne"], mine["offset"], mine["size"]) == (
                r["name"], r["type"], r["ne"], r["offset"], r["size"])
            assert mine["file_offset"] == ref["data_offset"] + r["offset"]
            assert g.tensor(r["name"])["offset"] == r["offset"]
        assert g.tensor("no.such.tensor") is None


def test_tensor_bytes_at_file_offset(files):
    """file_offset points at the tensor's bytes (the source map of Model::load)."""
    d, _ = files
    orc = Oracle()
    spec = {t[0]: t[3] for t in FX.fixtures(orc)["single"][0][2]}
    raw = (d / "moe_tiny.gguf").read_bytes()
    with ops.Gguf(d / "moe_tiny.gguf") as g:
        for t in g.tensors():
            assert raw[t["file_offset"]:t["file_offset"] + t["size"]] == spec[t["name"]], t["name"]


def test_shard_set(files):
    """"-00001-of-00002.gguf" opens both shards (core/model.cpp:400-423): KV of the
    first, tensors of both, each with its own shard's data offset."""
    d, _ = files
    gold = FX.golden()["files"]
    with ops.Gguf(d / "moe_split-00001-of-00002.gguf") as g:
        sh = g.shards()
        assert len(sh) == 2
        assert [s["data_offset"] for s in sh] == [gold["moe_split-00001-of-00002.gguf"]["data_offset"],
                                                   gold["moe_split-00002-of-00002.gguf"]["data_offset"]]
        assert [e["key"] for e in g.kv()] == [e["key"] for e in gold["moe_split-00001-of-00002.gguf"]["kv"]]
        ts = g.tensors()
        assert [t["shard"] for t in ts] == [0, 0, 1, 1]
        for t in ts:
            ref = gold[f"moe_split-0000{t['shard'] + 1}-of-00002.gguf"]
            r = next(x for x in ref["tensors"] if x["name"] == t["name"])
            assert t["file_offset"] == ref["data_offset"] + r["offset"]
        assert g.hparams()["n_layer"] == 1


def test_hparams_and_typed_lookups(files):
    """Model::load_hparams' keys with gguf_util's conversions: INT32 and UINT64 read
    as u32, FLOAT64 as f32; a missing or wrongly typed key gives the default."""
    d, _ = files
    with ops.Gguf(d / "moe_tiny.gguf") as g:
        hp = g.hparams()
        assert hp == {"arch": "qwen3moe", "n_layer": 2, "n_embd": FX.H, "n_expert": FX.E, "n_expert_used": FX.K_USED,
                      "n_ff_exp": FX.F_EXP, "expert_weights_scale": 1.0}
        assert g.get_u32("qwen3moe.expert_used_count") == FX.K_USED
        assert g.get_u32("test.i64") == (-(1 << 40)) & 0xFFFFFFFF
        assert g.get_u32("missing.key", 17) == 17
        assert g.get_u32("general.name", 5) == 5           # a string: default
        assert g.get_u32("test.u8", 9) == 9                # u8 is not one of the accepted types
        assert g.get_f32("test.f32") == 0.5
        assert g.get_f32("qwen3moe.expert_weights_scale") == 1.0
        assert g.get_f32("missing.key", 2.5) == 2.5
        assert g.get_str("general.architecture") == "qwen3moe"
        assert g.get_str("test.u8", "dflt") == "dflt"
        assert g.layer_bytes(0) > 0
        with pytest.raises(qa.QwmoeError):
            g.layer_bytes(2)


def test_malformed_files_rejected_like_the_reference(files, tmp_path):
    d, _ = files
    good = (d / "moe_tiny.gguf").read_bytes()
    gold = FX.golden()["malformed"]
    variants = FX.malformed_variants(good)
    assert set(variants) == set(gold)
    for name, data in variants.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        if gold[name]["reference_accepts"]:
            ops.Gguf(p).close()
        else:
            with pytest.raises(qa.QwmoeError) as e:
                ops.Gguf(p)
            assert e.value.status == QWMOE_ERR_FORMAT, name


def test_missing_file_and_truncated_data(files, tmp_path):
    with pytest.raises(qa.QwmoeError) as e:
        ops.Gguf(tmp_path / "absent.gguf")
    assert e.value.status == QWMOE_ERR_IO
    with pytest.raises(qa.QwmoeError) as e:   # a shard of the set is missing
        ops.Gguf(tmp_path / "x-00001-of-00002.gguf")
    assert e.value.status == QWMOE_ERR_IO


def test_open_handles_closed_at_exit(files):
    """A handle left open is freed by the library's exit hook (which Python
    runs before interpreter shutdown and the libraries' static destructors);
    a closed handle leaves the registry; a process that leaves one open exits
    cleanly."""
    import subprocess
    import sys
    d, _ = files
    g = ops.Gguf(d / "moe_tiny.gguf")
    assert g in ops._open_handles
    g2 = ops.Gguf(d / "moe_tiny.gguf")
    g2.close()
    assert g2 not in ops._open_handles and g2.h is None
    ops._close_open_handles()
    assert g.h is None and g not in ops._open_handles
    code = ("import sys; sys.path.insert(0, %r); from questwend_amd import ops; "
            "g = ops.Gguf(%r); print('open', bool(g.h))") % (str(qa.__file__.rsplit('/', 2)[0]), str(d / "moe_tiny.gguf"))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.strip() == "open True"
