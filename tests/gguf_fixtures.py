"""GGUF test fixtures (test infrastructure): deterministic content (seeded weights
quantized by the oracle, itself pinned to ggml byte for byte), written with
tests/gguf_writer.py.  tests/golden/gen_gguf.py pins these files against the
reference's own gguf writer and reader; tests regenerate them anywhere.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

import gguf_writer as W
from oracle_lib import F32, Q4_K, Q6_K, Q8_0, Oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "gguf_fixtures.json"
F16 = 1
H, E, K_USED, F_EXP = 256, 8, 2, 256   # E % 8 == 0, as the router requires


def _weights(orc: Oracle, t: int, rows: int, cols: int, seed: int) -> bytes:
    x = (np.random.default_rng(seed).standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if t == F32:
        return x.tobytes()
    return orc.quantize(t, x).tobytes()


def _layer_tensors(orc: Oracle, il: int, types, seed: int):
    tg, tu, td = types
    router = (np.random.default_rng(seed).standard_normal((E, H)) * 0.5).astype(np.float32)
    return [
        (f"blk.{il}.ffn_gate_inp.weight", F32, [H, E], router.tobytes()),
        (f"blk.{il}.ffn_gate_exps.weight", tg, [H, F_EXP, E], _weights(orc, tg, E * F_EXP, H, seed + 1)),
        (f"blk.{il}.ffn_up_exps.weight", tu, [H, F_EXP, E], _weights(orc, tu, E * F_EXP, H, seed + 2)),
        (f"blk.{il}.ffn_down_exps.weight", td, [F_EXP, H, E], _weights(orc, td, E * H, F_EXP, seed + 3)),
    ]


def fixtures(orc: Oracle) -> dict:
    """name -> list of files, each (file name, kvs, tensors, alignment)."""
    arch = "qwen3moe"
    base_kv = [
        ("general.architecture", W.STRING, arch),
        ("general.name", W.STRING, "qwmoe test fixture"),
    ]
    # the single-file model: 2 MoE layers, every KV type
    kv = base_kv + [
        (f"{arch}.block_count", W.U32, 2),
        (f"{arch}.embedding_length", W.U32, H),
        (f"{arch}.expert_count", W.U32, E),
        (f"{arch}.expert_used_count", W.I32, K_USED),            # INT32: converted like gguf_u32
        (f"{arch}.expert_feed_forward_length", W.U64, F_EXP),    # UINT64: converted like gguf_u32
        (f"{arch}.expert_weights_scale", W.F64, 1.0),            # FLOAT64: converted like gguf_f32
        ("tokenizer.ggml.tokens", W.ARRAY, ["a", "bc", "<|x|>", ""], W.STRING),
        ("tokenizer.ggml.token_type", W.ARRAY, [1, 1, 3, 2], W.I32),
        ("test.u8", W.U8, 7), ("test.i8", W.I8, -7), ("test.u16", W.U16, 65535), ("test.i16", W.I16, -3),
        ("test.f32", W.F32, 0.5), ("test.bool", W.BOOL, True), ("test.i64", W.I64, -(1 << 40)),
        ("test.f32s", W.ARRAY, [1.5, -2.25, 0.0], W.F32), ("test.empty", W.ARRAY, [], W.U8),
    ]
    emb = (np.random.default_rng(5).standard_normal((8, H))).astype(np.float16).tobytes()
    norm = np.ones(H, np.float32).tobytes()
    tensors = [("token_embd.weight", F16, [H, 8], emb)]
    tensors += _layer_tensors(orc, 0, (Q4_K, Q4_K, Q6_K), 100)
    tensors += _layer_tensors(orc, 1, (Q8_0, Q8_0, Q4_K), 200)
    tensors += [("output_norm.weight", F32, [H], norm)]
    single = [("moe_tiny.gguf", kv, tensors, 32)]
    # the same model with a non-default alignment ("general.alignment" = 64)
    a64 = [("moe_tiny_a64.gguf", kv[:2] + [("general.alignment", W.U32, 64)] + kv[2:], tensors, 64)]
    # a two-shard set: KV in the first shard, one layer's tensors split over both
    kv1 = base_kv + [
        (f"{arch}.block_count", W.U32, 1), (f"{arch}.embedding_length", W.U32, H),
        (f"{arch}.expert_count", W.U32, E), (f"{arch}.expert_used_count", W.U32, K_USED),
        (f"{arch}.expert_feed_forward_length", W.U32, F_EXP),
    ]
    lt = _layer_tensors(orc, 0, (Q4_K, Q4_K, Q4_K), 300)
    split = [("moe_split-00001-of-00002.gguf", kv1, lt[:2], 32),
             ("moe_split-00002-of-00002.gguf", [("general.architecture", W.STRING, arch)], lt[2:], 32)]
    return {"single": single, "a64": a64, "split": split}


# The reference writer pads to 32 bytes whatever "general.alignment" says (the
# key only takes effect when a file is read), so files with another alignment
# are pinned against the reference reader only.
WRITER_COMPARABLE = {"single", "split"}


def write_all(dst: Path, orc: Oracle) -> dict:
    """Writes every fixture file under dst; returns file name -> sha256."""
    dst.mkdir(parents=True, exist_ok=True)
    out = {}
    for files in fixtures(orc).values():
        for fname, kvs, tensors, align in files:
            data = W.write_gguf(dst / fname, kvs, tensors, alignment=align)
            out[fname] = hashlib.sha256(data).hexdigest()
    return out


def golden() -> dict:
    return json.loads(GOLDEN.read_text())


def raw_gguf(kvs: list[bytes], infos: list[tuple], data: bytes, alignment: int = 32, version: int = 3,
             n_tensors: int | None = None, n_kv: int | None = None) -> bytes:
    """A file from raw parts, for malformed variants: kvs are encoded KV pairs,
    infos are (name, n_dims, ne, type, offset)."""
    import struct
    out = b"GGUF" + struct.pack("<Iqq", version, len(infos) if n_tensors is None else n_tensors,
                                len(kvs) if n_kv is None else n_kv)
    out += b"".join(kvs)
    for name, n_dims, ne, t, off in infos:
        out += W._str(name) + struct.pack("<I", n_dims) + struct.pack(f"<{len(ne)}q", *ne) + struct.pack("<iQ", t, off)
    pad = (len(out) + alignment - 1) // alignment * alignment
    return out + b"\0" * (pad - len(out)) + data


def malformed_variants(good: bytes) -> dict:
    """name -> bytes: a valid file with one format rule broken.  The header's
    fields sit at fixed offsets (magic 0, version 4, n_tensors 8, n_kv 16)."""
    import struct
    arch = W.kv_bytes("general.architecture", W.STRING, "qwen3moe")
    f32 = lambda n: np.arange(n, dtype=np.float32).tobytes()  # noqa: E731
    ok_info = [("a.weight", 1, [8], F32, 0)]
    v = {
        "bad_magic": b"GGUX" + good[4:],
        "version_0": good[:4] + struct.pack("<I", 0) + good[8:],
        "version_1": good[:4] + struct.pack("<I", 1) + good[8:],
        "version_4": good[:4] + struct.pack("<I", 4) + good[8:],
        "version_swapped": good[:4] + struct.pack(">I", 3) + good[8:],
        "negative_n_tensors": good[:8] + struct.pack("<q", -1) + good[16:],
        "huge_n_kv": good[:16] + struct.pack("<q", 1 << 40) + good[24:],
        "truncated_header": good[:20],
        "truncated_metadata": good[:200],
        "empty_key": raw_gguf([W.kv_bytes("", W.U32, 1)], ok_info, f32(8)),
        "duplicate_key": raw_gguf([arch, arch], ok_info, f32(8)),
        "unknown_kv_type": raw_gguf([W._str("x") + struct.pack("<iI", 13, 0)], ok_info, f32(8)),
        "array_of_arrays": raw_gguf([W._str("x") + struct.pack("<iiQ", W.ARRAY, W.ARRAY, 0)], ok_info, f32(8)),
        "alignment_not_pow2": raw_gguf([W.kv_bytes("general.alignment", W.U32, 48)], ok_info, f32(8), alignment=48),
        "alignment_zero": raw_gguf([W.kv_bytes("general.alignment", W.U32, 0)], ok_info, f32(8)),
        "alignment_u64": raw_gguf([W.kv_bytes("general.alignment", W.U64, 32)], ok_info, f32(8)),
        "n_dims_5": raw_gguf([arch], [("a.weight", 5, [8, 1, 1, 1, 1], F32, 0)], f32(8)),
        "negative_ne": raw_gguf([arch], [("a.weight", 2, [8, -1], F32, 0)], f32(8)),
        "type_out_of_range": raw_gguf([arch], [("a.weight", 1, [8], 99, 0)], f32(8)),
        "type_removed": raw_gguf([arch], [("a.weight", 1, [32], 4, 0)], f32(8)),
        "row_not_whole_blocks": raw_gguf([arch], [("a.weight", 1, [100], Q4_K, 0)], bytes(144)),
        "offset_mismatch": raw_gguf([arch], [("a.weight", 1, [8], F32, 0), ("b.weight", 1, [8], F32, 64)], f32(16)),
        "duplicate_tensor": raw_gguf([arch], [("a.weight", 1, [8], F32, 0), ("a.weight", 1, [8], F32, 32)], f32(16)),
        "name_too_long": raw_gguf([arch], [("n" * 64, 1, [8], F32, 0)], f32(8)),
        "string_past_end": raw_gguf([W._str("x") + struct.pack("<iQ", W.STRING, 1 << 20)], [], b""),
        # valid metadata, data section cut short: opening succeeds (no data is read)
        "truncated_data": raw_gguf([arch], [("a.weight", 1, [64], F32, 0)], f32(8)),
    }
    return v
