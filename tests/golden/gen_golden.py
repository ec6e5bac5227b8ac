"""Writes the golden fixtures in tests/golden/ from the *real* ggml CPU backend.

The reference (kishida/questwend) ships no test vectors for this path, so the
vectors are produced here by running ggml itself: oracle/_ref/libqwref.so, built
by oracle/Makefile.ref from /root/reference/third_party/ggml sources (pinned ggml
commit 8e7f22b67ef4667b4ddd50230771287f328cfb3f), AVX2 configuration.  Only data
is committed: seeded inputs (or the seeds that regenerate them) and the
reference's outputs.

Run from the repository root:  python tests/golden/gen_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
from oracle_lib import (Q4_K, Q6_K, Q8_0, Q8_K, LayerWeights, Oracle, RefGGML, row_size,  # noqa: E402
                        vec_dot_type)


def special_rows(n: int, rng) -> list[np.ndarray]:
    """Inputs that exercise the quantizers' edge cases."""
    rows = []
    z = np.zeros(n, np.float32)
    rows.append(z.copy())                                   # all zero -> d = 0
    c = np.full(n, 0.0125, np.float32)
    rows.append(c)                                          # all equal
    neg = (rng.standard_normal(n) * 0.02).astype(np.float32)
    neg[7] = -0.2                                           # amax at a negative value
    rows.append(neg)
    tie = (rng.standard_normal(n) * 0.02).astype(np.float32)
    tie[3], tie[9] = -0.1, 0.1                              # equal |x|, first occurrence wins
    rows.append(tie)
    half = np.tile(np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 63.5], np.float32), n // 8)
    rows.append(half)                                       # exact .5 products
    big = (rng.standard_normal(n) * 1e3).astype(np.float32)
    rows.append(big)
    tiny = (rng.standard_normal(n) * 1e-6).astype(np.float32)
    rows.append(tiny)                                       # fp16 subnormal scales
    pos = np.abs(rng.standard_normal(n)).astype(np.float32) * np.float32(0.02)
    rows.append(pos)                                        # min > 0 branch of make_qkx2_quants
    return rows


def main() -> None:
    ref = RefGGML()
    orc = Oracle()
    rng = np.random.default_rng(20261201)
    out: dict[str, np.ndarray] = {}

    # ---- weight quantizers (ggml_quantize_chunk, imatrix NULL) ----
    n = 512
    base = [(rng.standard_normal(n) * 0.02).astype(np.float32) for _ in range(24)]
    Xw = np.stack(base + special_rows(n, rng))
    out["wq_x"] = Xw
    for t, name in ((Q8_0, "q8_0"), (Q4_K, "q4_K"), (Q6_K, "q6_K")):
        out[f"wq_{name}"] = ref.quantize(t, Xw).reshape(Xw.shape[0], -1)

    # ---- activation quantizers (type_traits_cpu from_float) ----
    acts = [rng.standard_normal(n).astype(np.float32) * np.float32(10 ** rng.uniform(-2, 2)) for _ in range(24)]
    Xa = np.stack(acts + special_rows(n, rng))
    out["aq_x"] = Xa
    for t, name in ((Q8_0, "q8_0"), (Q8_K, "q8_K")):
        q = np.stack([ref.from_float(t, r) for r in Xa])
        if t == Q8_K:
            # the reference leaves bsums unset for an all-zero block (ggml-quants.c:2781-2786);
            # store them as zero, which is what the kernels write
            blocks = q.reshape(Xa.shape[0], -1, 292)
            d = blocks[:, :, :4].copy().view(np.float32)[:, :, 0]
            blocks[d == 0, 260:] = 0
            q = blocks.reshape(Xa.shape[0], -1)
        out[f"aq_{name}"] = q

    # ---- block dot products on identical quantized inputs ----
    for t, name, K in ((Q4_K, "q4_K", 2048), (Q6_K, "q6_K", 1536), (Q8_0, "q8_0", 2048)):
        W = (rng.standard_normal((16, K)) * 0.02).astype(np.float32)
        X = rng.standard_normal((16, K)).astype(np.float32)
        wq = ref.quantize(t, W).reshape(16, -1)
        xq = np.stack([ref.from_float(vec_dot_type(t), x) for x in X])
        s = np.array([ref.vec_dot(t, K, wq[i], xq[i]) for i in range(16)], np.float32)
        out[f"dot_{name}_w"], out[f"dot_{name}_x"], out[f"dot_{name}_s"] = wq, xq, s

    # ---- router / softmax / argsort / swiglu / rms_norm single ops ----
    L = (rng.standard_normal((8, 128)) * 1.5).astype(np.float32)
    out["softmax_x"], out["softmax_y"] = L, ref.unary(0, L)
    out["argsort_y"] = ref.unary(1, out["softmax_y"])
    G = (rng.standard_normal((4, 768)) * 3).astype(np.float32)
    U = rng.standard_normal((4, 768)).astype(np.float32)
    out["swiglu_g"], out["swiglu_u"], out["swiglu_y"] = G, U, ref.unary(3, G, U)
    R = rng.standard_normal((4, 2048)).astype(np.float32)
    out["rms_x"], out["rms_y"] = R, ref.unary(2, R, param=1e-6)
    A = rng.standard_normal((8, 2048)).astype(np.float32)
    b = rng.standard_normal(2048).astype(np.float32)
    out["dotf32_a"], out["dotf32_b"], out["dotf32_y"] = A, b, ref.unary(4, A, b)
    A8 = rng.standard_normal((8, 8)).astype(np.float32)
    b8 = rng.standard_normal(8).astype(np.float32)
    out["dotf32k_a"], out["dotf32k_b"], out["dotf32k_y"] = A8, b8, ref.unary(4, A8, b8)

    # ---- small MoE layers (weights regenerate from the seed; hashes pin the bytes) ----
    cases = [("l_q4k", 512, 16, 4, 256, Q4_K, Q4_K, Q4_K, 11),
             ("l_q80", 512, 16, 4, 256, Q8_0, Q8_0, Q8_0, 12),
             ("l_mix", 512, 16, 4, 512, Q4_K, Q4_K, Q6_K, 13)]
    for name, H, E, k, F, tg, tu, td, seed in cases:
        lw = LayerWeights(H, E, k, F, tg, tu, td, seed=seed, oracle=orc)
        out[f"{name}_shape"] = np.array([H, E, k, F, tg, tu, td, seed], np.int64)
        h = hashlib.sha256()
        for arr in (lw.router.view(np.uint8), lw.gate, lw.up, lw.down):
            h.update(arr.tobytes())
        out[f"{name}_sha256"] = np.frombuffer(h.digest(), np.uint8)
        for T in (1, 5):
            x = np.random.default_rng(seed * 100 + T).standard_normal((T, H)).astype(np.float32)
            r = ref.layer(lw, T, rms_eps=1e-6)(x)
            out[f"{name}_T{T}_x"] = x
            for key in ("ids", "weights", "out", "xnext"):
                out[f"{name}_T{T}_{key}"] = r[key]

    # ---- grouping example (row order of ggml-cpu.c:1622-1637) ----
    # ggml keeps matrix_row_counts / matrix_rows in its work buffer, out of reach of
    # the public API, so this one is a brute-force restatement of those loops
    # (token outer, slot inner, append to the expert's list), not a ggml output.
    ids = np.stack([np.random.default_rng(t).permutation(16)[:4] for t in range(7)]).astype(np.int32)
    lists = [[] for _ in range(16)]
    for t in range(ids.shape[0]):
        for e in range(ids.shape[1]):
            lists[ids[t, e]].append((e, t))
    cnt = np.array([len(lst) for lst in lists], np.int32)
    off = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)
    rows = np.array([p for lst in lists for p in lst], np.int32)
    out["group_ids"], out["group_counts"], out["group_offsets"], out["group_rows"] = ids, cnt, off, rows

    path = HERE / "ggml_cpu_golden.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size / 1024:.1f} KiB, {len(out)} arrays)")


if __name__ == "__main__":
    main()
