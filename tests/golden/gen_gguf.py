"""Writes tests/golden/gguf_fixtures.json from the reference ggml's own gguf code.

For every fixture of tests/gguf_fixtures.py:
  1. the reference writer (gguf_init_empty / gguf_set_* / gguf_add_tensor /
     gguf_write_to_file, ggml/src/gguf.cpp) writes the same content, and the
     file must be byte-identical to the test writer's;
  2. the reference reader (gguf_init_from_file, no_alloc) reads it back, and
     its view -- version, alignment, data offset, every KV with its type and
     value, every tensor's name, type, ne, offset and size -- is recorded,
     together with the file's SHA-256.
It also records which malformed variants the reference reader rejects.

Runs only where the reference build exists (oracle/_ref/libqwref.so, built
from /root/reference by oracle/Makefile.ref); the JSON travels, the reference
does not.
"""
from __future__ import annotations

import ctypes as C
import json
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import gguf_fixtures as FX  # noqa: E402
import gguf_writer as W  # noqa: E402
from oracle_lib import REF_SO, Oracle  # noqa: E402


class InitParams(C.Structure):
    _fields_ = [("no_alloc", C.c_bool), ("ctx", C.c_void_p)]


class GgmlInitParams(C.Structure):
    _fields_ = [("mem_size", C.c_size_t), ("mem_buffer", C.c_void_p), ("no_alloc", C.c_bool)]


def load_ref():
    lib = C.CDLL(str(REF_SO))
    sig = {
        "gguf_init_empty": (C.c_void_p, []), "gguf_free": (None, [C.c_void_p]),
        "gguf_init_from_file": (C.c_void_p, [C.c_char_p, InitParams]),
        "gguf_write_to_file": (C.c_bool, [C.c_void_p, C.c_char_p, C.c_bool]),
        "gguf_get_version": (C.c_uint32, [C.c_void_p]), "gguf_get_alignment": (C.c_size_t, [C.c_void_p]),
        "gguf_get_data_offset": (C.c_size_t, [C.c_void_p]), "gguf_get_n_kv": (C.c_int64, [C.c_void_p]),
        "gguf_get_key": (C.c_char_p, [C.c_void_p, C.c_int64]), "gguf_get_kv_type": (C.c_int, [C.c_void_p, C.c_int64]),
        "gguf_get_arr_type": (C.c_int, [C.c_void_p, C.c_int64]), "gguf_get_arr_n": (C.c_size_t, [C.c_void_p, C.c_int64]),
        "gguf_get_arr_data": (C.c_void_p, [C.c_void_p, C.c_int64]),
        "gguf_get_arr_str": (C.c_char_p, [C.c_void_p, C.c_int64, C.c_size_t]),
        "gguf_get_val_data": (C.c_void_p, [C.c_void_p, C.c_int64]),
        "gguf_get_val_str": (C.c_char_p, [C.c_void_p, C.c_int64]),
        "gguf_get_n_tensors": (C.c_int64, [C.c_void_p]),
        "gguf_get_tensor_name": (C.c_char_p, [C.c_void_p, C.c_int64]),
        "gguf_get_tensor_type": (C.c_int, [C.c_void_p, C.c_int64]),
        "gguf_get_tensor_offset": (C.c_size_t, [C.c_void_p, C.c_int64]),
        "gguf_get_tensor_size": (C.c_size_t, [C.c_void_p, C.c_int64]),
        "gguf_get_tensor_ne": (C.POINTER(C.c_int64), [C.c_void_p, C.c_int64]),
        "gguf_set_val_str": (None, [C.c_void_p, C.c_char_p, C.c_char_p]),
        "gguf_set_arr_data": (None, [C.c_void_p, C.c_char_p, C.c_int, C.c_void_p, C.c_size_t]),
        "gguf_set_arr_str": (None, [C.c_void_p, C.c_char_p, C.POINTER(C.c_char_p), C.c_size_t]),
        "gguf_add_tensor": (None, [C.c_void_p, C.c_void_p]),
        "ggml_init": (C.c_void_p, [GgmlInitParams]), "ggml_free": (None, [C.c_void_p]),
        "ggml_new_tensor": (C.c_void_p, [C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_int64)]),
        "ggml_set_name": (C.c_void_p, [C.c_void_p, C.c_char_p]), "ggml_get_data": (C.c_void_p, [C.c_void_p]),
        "ggml_nbytes": (C.c_size_t, [C.c_void_p]),
    }
    for n, (r, a) in sig.items():
        f = getattr(lib, n)
        f.restype, f.argtypes = r, a
    scal = {W.U8: ("u8", C.c_uint8), W.I8: ("i8", C.c_int8), W.U16: ("u16", C.c_uint16), W.I16: ("i16", C.c_int16),
            W.U32: ("u32", C.c_uint32), W.I32: ("i32", C.c_int32), W.F32: ("f32", C.c_float),
            W.BOOL: ("bool", C.c_bool), W.U64: ("u64", C.c_uint64), W.I64: ("i64", C.c_int64),
            W.F64: ("f64", C.c_double)}
    for t, (nm, ct) in scal.items():
        f = getattr(lib, f"gguf_set_val_{nm}")
        f.restype, f.argtypes = None, [C.c_void_p, C.c_char_p, ct]
    return lib, scal


def ref_write(lib, scal, path, kvs, tensors, align):
    g = lib.gguf_init_empty()
    keep = []
    for kv in kvs:
        key, t, v = kv[0].encode(), kv[1], kv[2]
        if t == W.STRING:
            lib.gguf_set_val_str(g, key, v.encode())
        elif t == W.ARRAY:
            at = kv[3]
            if at == W.STRING:
                arr = (C.c_char_p * max(len(v), 1))(*[s.encode() for s in v])
                keep.append(arr)
                lib.gguf_set_arr_str(g, key, arr, len(v))
            else:
                ct = scal[at][1]
                arr = (ct * max(len(v), 1))(*v)
                keep.append(arr)
                lib.gguf_set_arr_data(g, key, at, C.cast(arr, C.c_void_p), len(v))
        else:
            getattr(lib, f"gguf_set_val_{scal[t][0]}")(g, key, v)
    mem = sum(len(d) for *_, d in tensors) + 1024 * (len(tensors) + 1) + (1 << 20)
    ctx = lib.ggml_init(GgmlInitParams(mem, None, False))
    for name, t, ne, data in tensors:
        ne_arr = (C.c_int64 * len(ne))(*ne)
        tt = lib.ggml_new_tensor(ctx, t, len(ne), ne_arr)
        lib.ggml_set_name(tt, name.encode())
        assert lib.ggml_nbytes(tt) == len(data)
        C.memmove(lib.ggml_get_data(tt), data, len(data))
        lib.gguf_add_tensor(g, tt)
    assert lib.gguf_write_to_file(g, str(path).encode(), False)
    lib.gguf_free(g)
    lib.ggml_free(ctx)


def ref_read(lib, path) -> dict | None:
    g = lib.gguf_init_from_file(str(path).encode(), InitParams(True, None))
    if not g:
        return None
    size = {W.U8: 1, W.I8: 1, W.U16: 2, W.I16: 2, W.U32: 4, W.I32: 4, W.F32: 4, W.BOOL: 1, W.U64: 8, W.I64: 8, W.F64: 8}
    fmt = {W.U8: "B", W.I8: "b", W.U16: "H", W.I16: "h", W.U32: "I", W.I32: "i", W.F32: "f", W.BOOL: "?",
           W.U64: "Q", W.I64: "q", W.F64: "d"}
    import struct
    kvs = []
    for i in range(lib.gguf_get_n_kv(g)):
        t = lib.gguf_get_kv_type(g, i)
        e = {"key": lib.gguf_get_key(g, i).decode(), "type": t}
        if t == W.ARRAY:
            at, n = lib.gguf_get_arr_type(g, i), lib.gguf_get_arr_n(g, i)
            e.update(arr_type=at, n=n)
            if at == W.STRING:
                e["value"] = [lib.gguf_get_arr_str(g, i, j).decode() for j in range(n)]
            else:
                raw = C.string_at(lib.gguf_get_arr_data(g, i), n * size[at]) if n else b""
                e["value"] = list(struct.unpack(f"<{n}{fmt[at]}", raw))
        elif t == W.STRING:
            e["value"] = lib.gguf_get_val_str(g, i).decode()
        else:
            e["value"] = struct.unpack("<" + fmt[t], C.string_at(lib.gguf_get_val_data(g, i), size[t]))[0]
        kvs.append(e)
    ts = []
    for i in range(lib.gguf_get_n_tensors(g)):
        ne = lib.gguf_get_tensor_ne(g, i)
        ts.append({"name": lib.gguf_get_tensor_name(g, i).decode(), "type": lib.gguf_get_tensor_type(g, i),
                   "ne": [ne[j] for j in range(4)], "offset": lib.gguf_get_tensor_offset(g, i),
                   "size": lib.gguf_get_tensor_size(g, i)})
    out = {"version": lib.gguf_get_version(g), "alignment": lib.gguf_get_alignment(g),
           "data_offset": lib.gguf_get_data_offset(g), "kv": kvs, "tensors": ts}
    lib.gguf_free(g)
    return out


def main():
    lib, scal = load_ref()
    orc = Oracle()
    out = {"files": {}, "malformed": {}}
    with tempfile.TemporaryDirectory() as td:
        td = Path(td)
        mine = FX.write_all(td / "mine", orc)
        (td / "ref").mkdir()
        for group, files in FX.fixtures(orc).items():
            for fname, kvs, tensors, align in files:
                a = (td / "mine" / fname).read_bytes()
                if group in FX.WRITER_COMPARABLE:
                    ref_write(lib, scal, td / "ref" / fname, kvs, tensors, align)
                    assert a == (td / "ref" / fname).read_bytes(), f"{fname}: the test writer and the reference writer differ"
                meta = ref_read(lib, td / "mine" / fname)
                assert meta is not None, f"{fname}: the reference reader rejects it"
                meta["sha256"] = mine[fname]
                meta["size"] = len(a)
                meta["reference_writer_identical"] = group in FX.WRITER_COMPARABLE
                out["files"][fname] = meta
                print(f"{fname}: {len(a)} bytes, read back by the reference reader"
                      + (", identical to the reference writer's" if group in FX.WRITER_COMPARABLE else ""), flush=True)
        good = (td / "mine" / "moe_tiny.gguf").read_bytes()
        for name, data in FX.malformed_variants(good).items():
            p = td / f"bad_{name}.gguf"
            p.write_bytes(data)
            out["malformed"][name] = {"reference_accepts": ref_read(lib, p) is not None}
    FX.GOLDEN.write_text(json.dumps(out, indent=1) + "\n")
    print("wrote", FX.GOLDEN)


if __name__ == "__main__":
    main()
