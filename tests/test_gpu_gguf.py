"""GPU tests of the GGUF MoE layer loader (qwmoe_gguf_load_moe_layer).

A layer loaded from a fixture file (written byte for byte as the reference's
gguf writer writes it; see tests/test_gguf.py) lands in device memory as the
file's bytes, and qwmoe_ffn_layer on it is bit-identical to the CPU oracle run
on the same tensors.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from questwend_amd import ops  # noqa: E402
import gguf_fixtures as FX  # noqa: E402
from oracle_lib import LayerWeights, Oracle  # noqa: E402

DEV = "cuda:0"


def note(msg: str) -> None:
    print(f"[gpu-gguf] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def lib_init():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    ops.init(0, 256 << 20)
    prev = ops.set_mfma_form(ops.MFMA_EXACT)   # bit-exact tests: heavy bins on the matrix cores replay ggml's float steps
    yield
    torch.cuda.synchronize()
    ops.set_mfma_form(prev)


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    d = tmp_path_factory.mktemp("gguf")
    FX.write_all(d, Oracle())
    return d


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def host_layer(g, il: int, raw_of) -> LayerWeights:
    """The oracle's view of layer il, built from the bytes the file holds."""
    hp = g.hparams()
    H, E, k, F = hp["n_embd"], hp["n_expert"], hp["n_expert_used"], hp["n_ff_exp"]
    names = [f"blk.{il}.ffn_gate_inp.weight", f"blk.{il}.ffn_gate_exps.weight", f"blk.{il}.ffn_up_exps.weight",
             f"blk.{il}.ffn_down_exps.weight"]
    infos = [g.tensor(n) for n in names]
    lw = LayerWeights.__new__(LayerWeights)
    lw.H, lw.E, lw.k, lw.F = H, E, k, F
    lw.type_gate, lw.type_up, lw.type_down = (t["type"] for t in infos[1:])
    lw.router = np.frombuffer(raw_of(infos[0]), np.float32).reshape(E, H).copy()
    lw.gate, lw.up, lw.down = (np.frombuffer(raw_of(t), np.uint8).copy() for t in infos[1:])
    lw.n_slots, lw.slot_of = E, None
    return lw, infos


@pytest.mark.parametrize("fname", ["moe_tiny.gguf", "moe_tiny_a64.gguf", "moe_split-00001-of-00002.gguf"])
def test_loaded_layers_equal_file_and_oracle(files, fname):
    orc = Oracle()
    shard_files = {}

    with ops.Gguf(files / fname) as g:
        paths = [files / fname] if "-of-" not in fname else [files / fname.replace("00001-of", f"0000{i + 1}-of")
                                                             for i in range(len(g.shards()))]

        def raw_of(t):
            if t["shard"] not in shard_files:
                shard_files[t["shard"]] = paths[t["shard"]].read_bytes()
            return shard_files[t["shard"]][t["file_offset"]:t["file_offset"] + t["size"]]

        for il in range(g.hparams()["n_layer"]):
            note(f"{fname} layer {il}")
            L, buf = g.load_layer(il, DEV)
            lw, infos = host_layer(g, il, raw_of)
            # device bytes: router, gate, up, down, each 256-byte aligned, as in the file
            dev_bytes = buf.cpu().numpy()
            off = 0
            for t in infos:
                assert dev_bytes[off:off + t["size"]].tobytes() == raw_of(t), t["name"]
                off += (t["size"] + 255) // 256 * 256
            assert (L.n_embd, L.n_expert, L.n_expert_used, L.n_ff) == (lw.H, lw.E, lw.k, lw.F)
            for T in (1, 3):
                x = np.random.default_rng(il * 10 + T).standard_normal((T, lw.H)).astype(np.float32)
                out, xn, ids, w = ops.ffn_layer(L, torch.from_numpy(x).to(DEV), rms_eps=1e-6)
                torch.cuda.synchronize()
                r = orc.moe_layer(lw, x, rms_eps=1e-6)
                assert np.array_equal(ids.cpu().numpy(), r["ids"]), (il, T)
                assert np.array_equal(bits(w.cpu().numpy()), bits(r["weights"])), (il, T)
                assert np.array_equal(bits(out.cpu().numpy()), bits(r["out"])), (il, T)
                assert np.array_equal(bits(xn.cpu().numpy()), bits(r["xnext"])), (il, T)
            assert ops.device_status(clear=True) == 0
            del buf


def test_load_errors(files, tmp_path):
    import questwend_amd as qa
    with ops.Gguf(files / "moe_tiny.gguf") as g:
        with pytest.raises(qa.QwmoeError):
            g.load_layer(5, DEV)                     # no such layer
    # metadata intact, data section cut short: opening works, loading reports an I/O error
    data = (files / "moe_tiny.gguf").read_bytes()
    p = tmp_path / "cut.gguf"
    p.write_bytes(data[:len(data) - 4096])
    with ops.Gguf(p) as g:
        with pytest.raises(qa.QwmoeError) as e:
            g.load_layer(1, DEV)
        assert e.value.status == -7
