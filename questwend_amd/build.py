"""Builds questwend_amd/libqwmoe.so (gfx950) with hipcc, in-tree.

    python -m questwend_amd.build        (or __graft_entry__.build())

Every HIP source is compiled with -ffp-contract=off (each fused multiply-add in
the kernels is written explicitly, which is what keeps the results
bit-identical to the reference CPU code) and with packed-fp32 instructions
disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libqwmoe.so"
ARCH = os.environ.get("QWMOE_ARCH", "gfx950")

SOURCES = ["quantize.hip", "router.hip", "mmid.hip", "mmid_mfma.hip", "ffn.hip", "decode.hip", "decode_xcd.hip", "decode_xcd_wide.hip", "verify_xcd.hip", "api.cpp", "slot_table.cpp", "gguf.cpp", "expert_cache.cpp", "slab_copy.hip", "layer_stack.cpp", "scratch.hip", "attn.hip", "gdn.hip"]

COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function",
          "-Wno-unused-variable", "-Wno-unused-but-set-variable"]
# v_dot4c_i32_i8 (dot6-insts) ties its accumulator to the destination, which
# costs a v_mov of 0 before every dot product that starts a sum; without it the
# compiler emits the VOP3P v_dot4_i32_i8 with an inline 0.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Xclang", "-target-feature", "-Xclang", "-dot6-insts"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    flags = COMMON + [f for f in DEVICE if f]
    if src.suffix == ".hip":
        cmd = [hipcc()] + flags + ["-x", "hip", "-c", str(src), "-o", str(obj)]
    else:
        cmd = [hipcc()] + flags + ["-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj, r.stderr


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in SOURCES if (CSRC / s).exists()]
    objs = [BUILD / (s.name + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(srcs))) as ex:
        for obj, err in ex.map(_compile, srcs, objs):
            if verbose and err.strip():
                print(err, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp)] + [str(o) for o in objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_ggml_backend()
    return LIB


# The ggml backend plugin (ggml_backend/ggml-qwmoe.cpp) compiles against the
# ggml headers of the tree it plugs into: QWMOE_GGML_DIR, by default the
# reference's vendored ggml.  It links libqwmoe.so; ggml's own symbols are left
# to the process's ggml, as for ggml's dynamically loaded backends.
GGML_DIR = Path(os.environ.get("QWMOE_GGML_DIR", "/root/reference/third_party/ggml"))
GGML_LIB = PKG / "libggml-qwmoe.so"


def build_ggml_backend() -> Path | None:
    if not (GGML_DIR / "src" / "ggml-backend-impl.h").exists():
        return None
    src = PKG / "ggml_backend" / "ggml-qwmoe.cpp"
    inc = PKG.parent / "include"
    tmp = GGML_LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-I{GGML_DIR / 'include'}",
           f"-I{GGML_DIR / 'src'}", f"-I{inc}", str(src), "-o", str(tmp), f"-L{PKG}", "-lqwmoe",
           "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"ggml backend build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, GGML_LIB)
    return GGML_LIB


if __name__ == "__main__":
    print(build(verbose=True))
