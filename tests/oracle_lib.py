"""ctypes bindings for the test oracles (test infrastructure only).

* ``Oracle``  -- oracle/liboracle.so, the CPU restatement of the reference path
  (oracle/qwmoe_oracle.cpp).
* ``RefGGML`` -- oracle/_ref/libqwref.so, the real ggml CPU backend compiled from
  /root/reference sources plus oracle/ref_driver.cpp.  Present only where it was
  built; tests that need it skip otherwise.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use these.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libqwref.so"
REF_SO_AVX512 = ROOT / "oracle" / "_ref" / "libqwref_avx512.so"   # ggml's AVX-512 branch (timed baseline)

F32, Q8_0, Q4_K, Q6_K, Q8_K, I32 = 0, 8, 12, 14, 15, 26
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292), F32: (1, 4)}


def row_size(t: int, n: int) -> int:
    qk, bs = BLOCK[t]
    assert n % qk == 0, (t, n)
    return n // qk * bs


def vec_dot_type(t: int) -> int:
    return Q8_0 if t == Q8_0 else Q8_K


def _p(a: np.ndarray | None):
    return None if a is None else C.c_void_p(a.ctypes.data)


class Oracle:
    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} not built (run make -C oracle)")
        L = self.lib = C.CDLL(str(path))
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_quantize.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64]
        L.orc_from_float.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64]
        L.orc_dequantize.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64]
        L.orc_vec_dot.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_dot_lanes.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_vec_dot_f32.restype = C.c_float
        L.orc_vec_dot_f32.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int]
        L.orc_v_expf.restype = C.c_float
        L.orc_v_expf.argtypes = [C.c_float]
        L.orc_rms_norm_mul.argtypes = [C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_float]
        L.orc_shared_expert_add.argtypes = ([C.c_int64, C.c_int64] + [C.c_int] * 3 + [C.c_void_p] * 5 + [C.c_int64]
                                            + [C.c_void_p] * 3)
        L.orc_v_expf_increases.restype = C.c_int64
        L.orc_v_expf_increases.argtypes = [C.c_uint32, C.c_uint32]
        L.orc_swiglu.argtypes = [C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_soft_max.argtypes = [C.c_int64, C.c_int64, C.c_void_p, C.c_void_p]
        L.orc_argsort_desc.argtypes = [C.c_int64, C.c_int64, C.c_void_p, C.c_void_p]
        L.orc_rms_norm.argtypes = [C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_float]
        L.orc_group_by_expert.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
                                          C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_mul_mat_id.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_size_t,
                                     C.c_size_t, C.c_int64, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p,
                                     C.c_int64, C.c_void_p, C.c_int64, C.c_void_p]
        L.orc_router.argtypes = [C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p,
                                 C.c_float, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_router_resident.argtypes = [C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p,
                                          C.c_float] + [C.c_void_p] * 6
        L.orc_moe_layer.argtypes = ([C.c_int64] * 5 + [C.c_int] * 3 + [C.c_void_p] * 4 + [C.c_int64]
                                    + [C.c_void_p] * 3 + [C.c_float, C.c_float] + [C.c_void_p] * 11)

    # -- quantization -------------------------------------------------------
    def quantize(self, t: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        n_per_row = x.shape[-1]
        nrows = x.size // n_per_row
        out = np.zeros(nrows * row_size(t, n_per_row), np.uint8)
        assert self.lib.orc_quantize(t, _p(x), _p(out), nrows, n_per_row) == 0
        return out

    def from_float(self, t: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(row_size(t, x.size), np.uint8)
        assert self.lib.orc_from_float(t, _p(x), _p(out), x.size) == 0
        return out

    def dequantize(self, t: int, q: np.ndarray, n: int) -> np.ndarray:
        out = np.zeros(n, np.float32)
        assert self.lib.orc_dequantize(t, _p(np.ascontiguousarray(q)), _p(out), n) == 0
        return out

    def vec_dot(self, t: int, n: int, xq: np.ndarray, yq: np.ndarray) -> np.float32:
        s = np.zeros(1, np.float32)
        self.lib.orc_vec_dot(t, n, _p(xq), _p(yq), _p(s))
        return s[0]

    def dot_lanes(self, t: int, n: int, xq: np.ndarray, yq: np.ndarray):
        nb = n // BLOCK[t][0]
        lanes = np.zeros((nb, 8), np.int32)
        mins = np.zeros((nb, 4), np.int32)
        assert self.lib.orc_dot_lanes(t, n, _p(xq), _p(yq), _p(lanes), _p(mins)) == 0
        return lanes, mins

    # -- float ops ------------------------------------------------------------
    def vec_dot_f32(self, x, y, tail_mode=2) -> float:
        x = np.ascontiguousarray(x, np.float32)
        y = np.ascontiguousarray(y, np.float32)
        return np.float32(self.lib.orc_vec_dot_f32(x.size, _p(x), _p(y), int(tail_mode)))

    def soft_max(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros_like(x)
        self.lib.orc_soft_max(x.shape[-1], x.size // x.shape[-1], _p(x), _p(y))
        return y

    def argsort_desc(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(x.shape, np.int32)
        self.lib.orc_argsort_desc(x.shape[-1], x.size // x.shape[-1], _p(x), _p(y))
        return y

    def rms_norm(self, x: np.ndarray, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros_like(x)
        self.lib.orc_rms_norm(x.shape[-1], x.size // x.shape[-1], _p(x), _p(y), eps)
        return y

    def rms_norm_mul(self, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        y = np.zeros_like(x)
        self.lib.orc_rms_norm_mul(x.shape[-1], x.size // x.shape[-1], _p(x), _p(w), _p(y), eps)
        return y

    def shared_expert_add(self, se: "SharedWeights", x, moe_out, resid=None) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        T, H = x.shape
        mo = np.ascontiguousarray(moe_out, np.float32)
        rs = None if resid is None else np.ascontiguousarray(resid, np.float32)
        out = np.zeros((T, H), np.float32)
        assert self.lib.orc_shared_expert_add(H, se.F, se.type_gate, se.type_up, se.type_down, _p(se.gate),
                                              _p(se.up), _p(se.down), _p(se.gate_inp), _p(x), T, _p(mo), _p(rs),
                                              _p(out)) == 0
        return out

    def swiglu(self, gate: np.ndarray, up: np.ndarray) -> np.ndarray:
        g = np.ascontiguousarray(gate, np.float32)
        u = np.ascontiguousarray(up, np.float32)
        y = np.zeros_like(g)
        # rows are independent; the AVX2 8-lane split restarts per row
        n = g.shape[-1]
        for r in range(g.size // n):
            self.lib.orc_swiglu(n, C.c_void_p(g.ctypes.data + 4 * r * n), C.c_void_p(u.ctypes.data + 4 * r * n),
                                C.c_void_p(y.ctypes.data + 4 * r * n))
        return y

    # -- path ----------------------------------------------------------------
    def group_by_expert(self, ids: np.ndarray, n_as: int):
        ids = np.ascontiguousarray(ids, np.int32)
        T, k = ids.shape
        counts = np.zeros(n_as, np.int32)
        offsets = np.zeros(n_as + 1, np.int32)
        rows = np.zeros((T * k, 2), np.int32)
        assert self.lib.orc_group_by_expert(_p(ids), k, T, k, n_as, _p(counts), _p(offsets), _p(rows)) == 0
        return counts, offsets, rows

    def mul_mat_id(self, t: int, K: int, N: int, n_as: int, w: np.ndarray, b: np.ndarray,
                   ids: np.ndarray, slot_of: np.ndarray | None = None, n_logical: int = 0) -> np.ndarray:
        """b: f32 [T, b_ne1, K]; ids: i32 [T, k] -> dst f32 [T, k, N]."""
        b = np.ascontiguousarray(b, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        T, b_ne1, _ = b.shape
        k = ids.shape[1]
        rs = row_size(t, K)
        dst = np.zeros((T, k, N), np.float32)
        so = None if slot_of is None else np.ascontiguousarray(slot_of, np.int32)
        rc = self.lib.orc_mul_mat_id(t, K, N, n_as, _p(w), rs, rs * N, b_ne1, T, _p(b), k, _p(ids), k,
                                     _p(so), n_logical, _p(dst))
        assert rc == 0
        return dst

    def router(self, W: np.ndarray, x: np.ndarray, k: int, scale: float = 0.0):
        E, H = W.shape
        x = np.ascontiguousarray(x, np.float32).reshape(-1, H)
        T = x.shape[0]
        ids = np.zeros((T, k), np.int32)
        w = np.zeros((T, k), np.float32)
        logits = np.zeros((T, E), np.float32)
        probs = np.zeros((T, E), np.float32)
        self.lib.orc_router(H, E, k, T, _p(np.ascontiguousarray(W, np.float32)), _p(x), scale, _p(ids),
                            _p(w), _p(logits), _p(probs))
        return ids, w, logits, probs

    def router_resident(self, W: np.ndarray, x: np.ndarray, k: int, mask: np.ndarray | None, scale: float = 0.0):
        """Resident-only routing: returns ids, weights, want (the unmasked top k), probs."""
        E, H = W.shape
        x = np.ascontiguousarray(x, np.float32).reshape(-1, H)
        T = x.shape[0]
        ids = np.zeros((T, k), np.int32)
        w = np.zeros((T, k), np.float32)
        want = np.zeros((T, k), np.int32)
        probs = np.zeros((T, E), np.float32)
        m = None if mask is None else np.ascontiguousarray(mask, np.float32)
        self.lib.orc_router_resident(H, E, k, T, _p(np.ascontiguousarray(W, np.float32)), _p(x), scale, _p(m),
                                     _p(want), _p(ids), _p(w), None, _p(probs))
        return ids, w, want, probs

    def moe_layer(self, layer: "LayerWeights", x: np.ndarray, rms_eps: float = -1.0, scale: float = 0.0,
                  resmask: np.ndarray | None = None):
        """resmask: f32 [E] (0 / -inf) for resident-only routing; the result then
        also holds 'want', the unmasked top k."""
        H, E, k, F = layer.H, layer.E, layer.k, layer.F
        x = np.ascontiguousarray(x, np.float32).reshape(-1, H)
        T = x.shape[0]
        out = np.zeros((T, H), np.float32)
        xnext = np.zeros((T, H), np.float32)
        ids = np.zeros((T, k), np.int32)
        w = np.zeros((T, k), np.float32)
        gate = np.zeros((T, k, F), np.float32)
        up = np.zeros((T, k, F), np.float32)
        act = np.zeros((T, k, F), np.float32)
        ex = np.zeros((T, k, H), np.float32)
        sg, su, sd = (None, None, None) if layer.slot_of is None else layer.slot_of
        m = None if resmask is None else np.ascontiguousarray(resmask, np.float32)
        want = np.zeros((T, k), np.int32)
        rc = self.lib.orc_moe_layer(H, E, k, F, T, layer.type_gate, layer.type_up, layer.type_down,
                                    _p(layer.router), _p(layer.gate), _p(layer.up), _p(layer.down),
                                    layer.n_slots, _p(sg), _p(su), _p(sd), scale, rms_eps, _p(x), _p(out),
                                    _p(xnext), _p(ids), _p(w), _p(gate), _p(up), _p(act), _p(ex), _p(m),
                                    _p(want) if m is not None else None)
        assert rc == 0
        r = dict(out=out, xnext=xnext, ids=ids, weights=w, gate=gate, up=up, act=act, experts=ex)
        if m is not None:
            r["want"] = want
        return r


class LayerWeights:
    """One MoE layer's synthetic weights, quantized on the CPU.

    gate/up: [n_slots] matrices of F rows x H; down: [n_slots] matrices of H rows x F.
    With ``permute`` the logical experts are stored at a seeded random slot
    permutation and ``slot_of`` holds the (gate, up, down) logical->slot tables.
    """

    def __init__(self, H, E, k, F, type_gate=Q4_K, type_up=Q4_K, type_down=Q4_K, seed=0,
                 oracle: Oracle | None = None, permute=False, zipf_skew: float = 0.0):
        self.H, self.E, self.k, self.F = H, E, k, F
        self.type_gate, self.type_up, self.type_down = type_gate, type_up, type_down
        rng = np.random.default_rng(seed)
        orc = oracle or Oracle()
        self.router = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        if zipf_skew > 0:
            self.router *= zipf_row_scales(E, zipf_skew)[:, None]
        wg = rng.standard_normal((E, F, H), dtype=np.float32) * np.float32(0.02)
        wu = rng.standard_normal((E, F, H), dtype=np.float32) * np.float32(0.02)
        wd = rng.standard_normal((E, H, F), dtype=np.float32) * np.float32(0.02)
        self.n_slots = E
        self.slot_of = None
        qg = orc.quantize(type_gate, wg.reshape(-1, H)).reshape(E, -1)
        qu = orc.quantize(type_up, wu.reshape(-1, H)).reshape(E, -1)
        qd = orc.quantize(type_down, wd.reshape(-1, F)).reshape(E, -1)
        if permute:
            perms = [rng.permutation(E).astype(np.int32) for _ in range(3)]
            pools = []
            for q, p in zip((qg, qu, qd), perms):
                pool = np.empty_like(q)
                pool[p] = q          # logical expert e lives in slot p[e]
                pools.append(pool)
            qg, qu, qd = pools
            self.slot_of = tuple(perms)
        self.gate = np.ascontiguousarray(qg.reshape(-1))
        self.up = np.ascontiguousarray(qu.reshape(-1))
        self.down = np.ascontiguousarray(qd.reshape(-1))


def zipf_row_scales(E: int, s: float, k: int = 8, T: int = 512) -> np.ndarray:
    """The benchmark's configs[2] skew (bench.zipf_router_scales): router row
    scales under which expert popularity follows a Zipf(s) rank profile."""
    import sys
    sys.path.insert(0, str(ROOT))
    from bench import zipf_router_scales
    return zipf_router_scales(E, k, s, T)


class SharedWeights:
    """A shared expert's weights, seeded: gate / up [F, H] and down [H, F]
    quantized from N(0, 0.02) fp32, gate_inp f32 [H] N(0, 0.02) (blk.N.ffn_*_shexp)."""

    def __init__(self, H, F, type_gate, type_up, type_down, seed, oracle: Oracle):
        rng = np.random.default_rng(seed)
        self.H, self.F = H, F
        self.type_gate, self.type_up, self.type_down = type_gate, type_up, type_down
        self.gate = oracle.quantize(type_gate, (rng.standard_normal((F, H)) * 0.02).astype(np.float32))
        self.up = oracle.quantize(type_up, (rng.standard_normal((F, H)) * 0.02).astype(np.float32))
        self.down = oracle.quantize(type_down, (rng.standard_normal((H, F)) * 0.02).astype(np.float32))
        self.gate_inp = (rng.standard_normal(H) * 0.02).astype(np.float32)


class AttnWeights:
    """A Qwen3 attention block's weights, seeded: attn_q [n_head * D, H],
    attn_k / attn_v [n_head_kv * D, H], attn_output [H, n_head * D] quantized
    from N(0, 0.02) fp32 (types (q, k, v, o)); the f32 norms N(1, 0.1)."""

    def __init__(self, H, n_head, n_head_kv, D, types, seed, oracle: Oracle, freq_base=1e6):
        rng = np.random.default_rng(seed)
        self.H, self.n_head, self.n_head_kv, self.D, self.types, self.freq_base = H, n_head, n_head_kv, D, types, freq_base
        NQ, NK = n_head * D, n_head_kv * D
        q = lambda t, r, c: oracle.quantize(t, (rng.standard_normal((r, c)) * 0.02).astype(np.float32))  # noqa: E731
        self.wq, self.wk, self.wv = q(types[0], NQ, H), q(types[1], NK, H), q(types[2], NK, H)
        self.wo = q(types[3], H, NQ)
        nrm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)  # noqa: E731
        self.attn_norm, self.ffn_norm, self.q_norm, self.k_norm = nrm(H), nrm(H), nrm(D), nrm(D)


def attn_seg_restated(aw: AttnWeights, h, n_past: int, k_cache, v_cache, orc: Oracle, eps: float = 1e-6):
    """Seg A's attention half (core/runtime.cpp:1976-2030, build_attn 681-734)
    restated on the CPU: the projections are the oracle's quantized mul_mat (ggml's
    row dots, bit for bit); the norms follow ggml_rms_norm (double sum); RoPE NEOX
    with ggml_rope_cache_init's theta_{i+1} = theta_i * powf(base, -2/n_rot) in
    fp32; K, V rounded to f16 into the caches; Q and the probabilities rounded to
    f16 (the f16 mul_mat's vec_dot_type); the products and the softmax in float64.
    Returns (attn_resid, ffn_in, q_roped, att); the caches are updated in place."""
    h = np.ascontiguousarray(h, np.float32)
    T, H = h.shape
    nq, nk, D = aw.n_head, aw.n_head_kv, aw.D
    R, NQ, NK = nq // nk, nq * D, nk * D

    def mm(t, w, x, N):
        return orc.mul_mat_id(t, x.shape[1], N, 1, w, x[:, None, :], np.zeros((x.shape[0], 1), np.int32))[:, 0, :]

    cur = orc.rms_norm_mul(h, aw.attn_norm, eps)
    Q = mm(aw.types[0], aw.wq, cur, NQ).reshape(T, nq, D)
    K = mm(aw.types[1], aw.wk, cur, NK).reshape(T, nk, D)
    V = mm(aw.types[2], aw.wv, cur, NK).reshape(T, nk, D)
    Q = orc.rms_norm_mul(Q.reshape(-1, D), aw.q_norm, eps).reshape(T, nq, D)
    K = orc.rms_norm_mul(K.reshape(-1, D), aw.k_norm, eps).reshape(T, nk, D)
    scale = np.float32(np.power(np.float32(aw.freq_base), np.float32(-2.0) / np.float32(D), dtype=np.float32))
    half = D // 2

    def rope(x, pos):
        th = np.zeros(half, np.float32)
        t_ = np.float32(pos)
        for i in range(half):
            th[i] = t_
            t_ = np.float32(t_ * scale)
        c = np.cos(th.astype(np.float64)).astype(np.float32)
        s_ = np.sin(th.astype(np.float64)).astype(np.float32)
        x0, x1 = x[..., :half], x[..., half:]
        return np.concatenate([x0 * c - x1 * s_, x0 * s_ + x1 * c], axis=-1).astype(np.float32)

    Q = np.stack([rope(Q[t], n_past + t) for t in range(T)])
    K = np.stack([rope(K[t], n_past + t) for t in range(T)])
    k_cache[n_past:n_past + T] = K.reshape(T, NK).astype(np.float16).view(np.uint16)
    v_cache[n_past:n_past + T] = V.reshape(T, NK).astype(np.float16).view(np.uint16)
    n_kv = n_past + T
    Kc = k_cache[:n_kv].view(np.float16).astype(np.float64).reshape(n_kv, nk, D)
    Vc = v_cache[:n_kv].view(np.float16).astype(np.float64).reshape(n_kv, nk, D)
    att = np.zeros((T, nq, D), np.float32)
    kq_scale = np.float32(1.0 / np.sqrt(np.float32(D)))
    for t in range(T):
        for hh in range(nq):
            g = hh // R
            q16 = Q[t, hh].astype(np.float16).astype(np.float64)
            sc = (Kc[:, g, :] @ q16).astype(np.float32) * kq_scale
            sc[n_past + t + 1:] = -np.inf
            e = np.exp(sc.astype(np.float64) - sc.max())
            p = (e / e.sum()).astype(np.float32).astype(np.float16).astype(np.float64)
            att[t, hh] = (p @ Vc[:, g, :]).astype(np.float32)
    att = att.reshape(T, NQ)
    proj = mm(aw.types[3], aw.wo, att, H)
    resid = (proj + h).astype(np.float32)
    fin = orc.rms_norm_mul(resid, aw.ffn_norm, eps)
    return resid, fin, Q.reshape(T, NQ), att


class GdnWeights:
    """A gated-delta-net block's weights (qwen3next / qwen35moe recurrent
    layers), seeded: attn_qkv [conv_ch, H], attn_gate [d_inner, H], ssm_beta and
    ssm_alpha [H_v, H], ssm_out [H, d_inner] quantized from N(0, 0.02) fp32
    (types (qkv, gate, beta, alpha, out)); conv1d [conv_ch][d_conv] N(0, 0.3);
    dt_bias N(0, 0.5); ssm_a = -U(0.5, 2) (decays below 1); the f32 norms
    N(1, 0.1).  d_inner = H_v * S, conv_ch = d_inner + 2 H_k S."""

    def __init__(self, H, S, H_k, H_v, d_conv, types, seed, oracle: Oracle):
        rng = np.random.default_rng(seed)
        self.H, self.S, self.H_k, self.H_v, self.d_conv, self.types = H, S, H_k, H_v, d_conv, types
        self.d_inner, self.key_dim = H_v * S, H_k * S
        self.conv_ch = self.d_inner + 2 * self.key_dim
        q = lambda t, r, c: oracle.quantize(t, (rng.standard_normal((r, c)) * 0.02).astype(np.float32))  # noqa: E731
        self.w_qkv, self.w_gate = q(types[0], self.conv_ch, H), q(types[1], self.d_inner, H)
        self.w_beta, self.w_alpha = q(types[2], H_v, H), q(types[3], H_v, H)
        self.w_out = q(types[4], H, self.d_inner)
        self.conv1d = (rng.standard_normal((self.conv_ch, d_conv)) * 0.3).astype(np.float32)
        self.dt_bias = (rng.standard_normal(H_v) * 0.5).astype(np.float32)
        self.ssm_a = (-rng.uniform(0.5, 2.0, H_v)).astype(np.float32)
        nrm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)  # noqa: E731
        self.attn_norm, self.ffn_norm, self.ssm_norm = nrm(H), nrm(H), nrm(S)

    def fresh_state(self, rng=None):
        """(conv_state f32 [conv_ch][d_conv - 1], ssm_state f32 [H_v][S][S]):
        zeros, or small seeded values when rng is given."""
        if rng is None:
            return (np.zeros((self.conv_ch, self.d_conv - 1), np.float32),
                    np.zeros((self.H_v, self.S, self.S), np.float32))
        return ((rng.standard_normal((self.conv_ch, self.d_conv - 1)) * 0.5).astype(np.float32),
                (rng.standard_normal((self.H_v, self.S, self.S)) * 0.05).astype(np.float32))


def gdn_seg_restated(gw: GdnWeights, h, conv_state, ssm_state, orc: Oracle, eps: float = 1e-6):
    """Seg A's recurrent half (core/runtime.cpp:1976-1995 with build_gdn 737-859)
    restated on the CPU: the projections are the oracle's quantized mul_mat
    (ggml's row dots, bit for bit); rms_norm and l2_norm with ggml's double sums;
    sigmoid / softplus (threshold 20) / silu in float32 as ggml's unary ops;
    ggml_ssm_conv's window dot in float32; ggml_gated_delta_net's recurrence
    (ops.cpp:10734-10887: per value head h with key head h % H_k, the state
    M = S^T, M *= exp(g); delta = (v - M k) beta; M += delta k^T; out = M q / sqrt(S))
    in float64.  Returns (attn_resid, ffn_in, gated_out); conv_state and
    ssm_state are updated in place."""
    h = np.ascontiguousarray(h, np.float32)
    T, H = h.shape
    S, Hk, Hv, dc = gw.S, gw.H_k, gw.H_v, gw.d_conv
    d_inner, key_dim, conv_ch = gw.d_inner, gw.key_dim, gw.conv_ch
    f32 = np.float32

    def mm(t, w, x, N):
        return orc.mul_mat_id(t, x.shape[1], N, 1, w, x[:, None, :], np.zeros((x.shape[0], 1), np.int32))[:, 0, :]

    cur = orc.rms_norm_mul(h, gw.attn_norm, eps)
    qkv = mm(gw.types[0], gw.w_qkv, cur, conv_ch)
    z = mm(gw.types[1], gw.w_gate, cur, d_inner)
    braw = mm(gw.types[2], gw.w_beta, cur, Hv)
    beta = (f32(1.0) / (f32(1.0) + np.exp(-braw).astype(f32))).astype(f32)
    a = (mm(gw.types[3], gw.w_alpha, cur, Hv) + gw.dt_bias).astype(f32)
    sp = np.where(a > f32(20.0), a, np.log(f32(1.0) + np.exp(a).astype(f32)).astype(f32)).astype(f32)
    g = (sp * gw.ssm_a).astype(f32)
    # causal conv over [conv_state | qkv^T], d_conv taps, float32 in tap order
    inp = np.concatenate([conv_state, qkv.T], axis=1).astype(f32)          # [conv_ch, dc - 1 + T]
    conv = np.zeros((T, conv_ch), f32)
    for t in range(T):
        acc = np.zeros(conv_ch, f32)
        for j in range(dc):
            acc = (acc + inp[:, t + j] * gw.conv1d[:, j]).astype(f32)
        conv[t] = acc
    conv_state[:] = inp[:, T:T + dc - 1]
    conv = (conv.astype(np.float64) / (1.0 + np.exp(-conv.astype(np.float64)))).astype(f32)

    def l2(x):
        ss = np.sum((x * x).astype(np.float64), axis=-1, keepdims=True)
        return (x * (f32(1.0) / np.maximum(np.sqrt(ss).astype(f32), f32(eps)))).astype(f32)

    q = l2(conv[:, :key_dim].reshape(T, Hk, S)).astype(np.float64)
    k = l2(conv[:, key_dim:2 * key_dim].reshape(T, Hk, S)).astype(np.float64)
    v = conv[:, 2 * key_dim:].reshape(T, Hv, S).astype(np.float64)
    M = ssm_state.astype(np.float64)                                        # [Hv][j][i] = S[i][j]
    o = np.zeros((T, Hv, S), np.float64)
    scale = 1.0 / np.sqrt(np.float32(S))
    for t in range(T):
        for hv in range(Hv):
            hk = hv % Hk
            M[hv] *= np.exp(np.float64(g[t, hv]))
            delta = (v[t, hv] - M[hv] @ k[t, hk]) * np.float64(beta[t, hv])
            M[hv] += np.outer(delta, k[t, hk])
            o[t, hv] = (M[hv] @ q[t, hk]) * scale
    ssm_state[:] = M.astype(f32)
    o = o.astype(f32)
    ss = np.sum((o * o).astype(np.float64), axis=-1, keepdims=True)
    sc = (f32(1.0) / np.sqrt((ss / S).astype(f32) + f32(eps))).astype(f32)
    zz = z.reshape(T, Hv, S).astype(np.float64)
    silu_z = (zz / (1.0 + np.exp(-zz))).astype(f32)
    y = ((o * sc).astype(f32) * gw.ssm_norm).astype(f32)
    y = (y * silu_z).astype(f32).reshape(T, d_inner)
    proj = mm(gw.types[4], gw.w_out, y, H)
    resid = (proj + h).astype(f32)
    fin = orc.rms_norm_mul(resid, gw.ffn_norm, eps)
    return resid, fin, y


class RefGGML:
    def __init__(self, path: Path = REF_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} not built (run make -C oracle ref)")
        L = self.lib = C.CDLL(str(path))
        L.qwref_quantize.restype = C.c_size_t
        L.qwref_quantize.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64]
        L.qwref_from_float.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64]
        L.qwref_vec_dot.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
        L.qwref_dequantize.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64]
        L.qwref_layer_create.restype = C.c_void_p
        L.qwref_layer_create.argtypes = ([C.c_int64] * 5 + [C.c_int] * 3 + [C.c_void_p] * 4
                                         + [C.c_float, C.c_float, C.c_int])
        L.qwref_layer_free.argtypes = [C.c_void_p]
        L.qwref_layer_eval.argtypes = [C.c_void_p] + [C.c_void_p] * 11 + [C.c_int]
        L.qwref_mul_mat_id.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_int64,
                                       C.c_int64, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p, C.c_int]
        L.qwref_unary.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_float,
                                  C.c_void_p, C.c_int]
        L.qwref_stack_run.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_void_p, C.c_int]
        L.qwref_isa.restype = C.c_int
        L.qwref_shared_expert_add.argtypes = ([C.c_int64, C.c_int64, C.c_int64] + [C.c_int] * 3 + [C.c_void_p] * 8
                                              + [C.c_int])
        L.qwref_router_resident.argtypes = ([C.c_int64] * 4 + [C.c_void_p] * 3 + [C.c_float] + [C.c_void_p] * 4
                                            + [C.c_int])
        L.qwref_gdn_seg.argtypes = ([C.c_int64] * 5 + [C.c_float, C.c_int64] + [C.c_void_p] * 2
                                    + [C.c_int, C.c_void_p] * 4 + [C.c_void_p] * 4 + [C.c_int, C.c_void_p]
                                    + [C.c_void_p] * 6 + [C.c_int])
        L.qwref_attn_seg.argtypes = ([C.c_int64] * 5 + [C.c_float] * 2 + [C.c_int64] * 3 + [C.c_void_p] * 2
                                     + [C.c_int, C.c_void_p] * 4 + [C.c_void_p] * 9 + [C.c_int])

    def attn_seg(self, aw, h, n_past: int, k_cache, v_cache, eps: float = 1e-6, n_threads: int = 4):
        """ggml's Seg A attention half (build_segA + build_attn, manual path) on
        AttnWeights aw: (attn_resid, ffn_in, q_roped, att); k_cache / v_cache
        (uint16 [n_ctx, n_head_kv * D]) are updated in place."""
        h = np.ascontiguousarray(h, np.float32)
        T, H = h.shape
        NQ = aw.n_head * aw.D
        resid, fin = np.zeros((T, H), np.float32), np.zeros((T, H), np.float32)
        qo, att = np.zeros((T, NQ), np.float32), np.zeros((T, NQ), np.float32)
        assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
        rc = self.lib.qwref_attn_seg(H, aw.n_head, aw.n_head_kv, aw.D, aw.D, aw.freq_base, eps, T, n_past,
                                     k_cache.shape[0], _p(h), _p(aw.attn_norm), aw.types[0], _p(aw.wq), aw.types[1],
                                     _p(aw.wk), aw.types[2], _p(aw.wv), aw.types[3], _p(aw.wo), _p(aw.q_norm),
                                     _p(aw.k_norm), _p(aw.ffn_norm), _p(k_cache), _p(v_cache), _p(resid), _p(fin),
                                     _p(qo), _p(att), n_threads)
        assert rc == 0, rc
        return resid, fin, qo, att

    def gdn_seg(self, gw, h, conv_state, ssm_state, eps: float = 1e-6, n_threads: int = 4):
        """ggml's Seg A recurrent half (build_segA + build_gdn) on GdnWeights gw:
        (attn_resid, ffn_in, gated_out); conv_state / ssm_state are updated in place."""
        h = np.ascontiguousarray(h, np.float32)
        T, H = h.shape
        resid, fin = np.zeros((T, H), np.float32), np.zeros((T, H), np.float32)
        y = np.zeros((T, gw.d_inner), np.float32)
        assert conv_state.flags.c_contiguous and ssm_state.flags.c_contiguous
        assert conv_state.dtype == np.float32 and ssm_state.dtype == np.float32
        t = gw.types
        rc = self.lib.qwref_gdn_seg(H, gw.S, gw.H_k, gw.H_v, gw.d_conv, eps, T, _p(h), _p(gw.attn_norm), t[0],
                                    _p(gw.w_qkv), t[1], _p(gw.w_gate), t[2], _p(gw.w_beta), t[3], _p(gw.w_alpha),
                                    _p(gw.dt_bias), _p(gw.ssm_a), _p(gw.conv1d), _p(gw.ssm_norm), t[4],
                                    _p(gw.w_out), _p(gw.ffn_norm), _p(conv_state), _p(ssm_state), _p(resid),
                                    _p(fin), _p(y), n_threads)
        assert rc == 0, rc
        return resid, fin, y

    def router_resident(self, W, x, k: int, mask, scale: float = 0.0, n_threads: int = 2):
        """ggml's resident-only router: ids, weights, want (unmasked top k), probs."""
        E, H = W.shape
        x = np.ascontiguousarray(x, np.float32).reshape(-1, H)
        T = x.shape[0]
        ids = np.zeros((T, k), np.int32)
        w = np.zeros((T, k), np.float32)
        want = np.zeros((T, k), np.int32)
        probs = np.zeros((T, E), np.float32)
        assert self.lib.qwref_router_resident(H, E, k, T, _p(np.ascontiguousarray(W, np.float32)), _p(x),
                                              _p(np.ascontiguousarray(mask, np.float32)), scale, _p(want), _p(ids),
                                              _p(w), _p(probs), n_threads) == 0
        return ids, w, want, probs

    def shared_expert_add(self, se: SharedWeights, x, moe_out, resid=None, n_threads=4):
        x = np.ascontiguousarray(x, np.float32)
        T, H = x.shape
        mo = np.ascontiguousarray(moe_out, np.float32)
        rs = None if resid is None else np.ascontiguousarray(resid, np.float32)
        out = np.zeros((T, H), np.float32)
        assert self.lib.qwref_shared_expert_add(H, se.F, T, se.type_gate, se.type_up, se.type_down, _p(se.gate),
                                                _p(se.up), _p(se.down), _p(se.gate_inp), _p(x), _p(mo), _p(rs),
                                                _p(out), n_threads) == 0
        return out

    def isa(self) -> int:
        """512: this build takes ggml's AVX-512 branch; 256: AVX2."""
        return self.lib.qwref_isa()

    def stack_run(self, layers, xs, n_warmup: int, n_threads: int, want_ids=True):
        """Layers (RefLayer, T = 1, each with an RMSNorm) chained on the tokens
        xs [n_warmup + n_steps, H]: per timed step the seconds (steady_clock),
        the last layer's output, every layer's ids and top-k margins."""
        xs = np.ascontiguousarray(xs, np.float32)
        n_steps = xs.shape[0] - n_warmup
        H, k, nl = layers[0].lw.H, layers[0].lw.k, len(layers)
        hs = (C.c_void_p * nl)(*[r.h for r in layers])
        out = np.zeros((n_steps, H), np.float32)
        ids = np.zeros((n_steps, nl, k), np.int32) if want_ids else None
        margin = np.zeros((n_steps, nl), np.float32) if want_ids else None
        step_s = np.zeros(n_steps, np.float64)
        rc = self.lib.qwref_stack_run(hs, nl, _p(xs), n_warmup, n_steps, _p(out), _p(ids), _p(margin), _p(step_s),
                                      n_threads)
        assert rc == 0
        return dict(out=out, ids=ids, margin=margin, step_s=step_s)

    def quantize(self, t, x):
        x = np.ascontiguousarray(x, np.float32)
        n_per_row = x.shape[-1]
        nrows = x.size // n_per_row
        out = np.zeros(nrows * row_size(t, n_per_row), np.uint8)
        self.lib.qwref_quantize(t, _p(x), _p(out), nrows, n_per_row)
        return out

    def from_float(self, t, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(row_size(t, x.size), np.uint8)
        assert self.lib.qwref_from_float(t, _p(x), _p(out), x.size) == 0
        return out

    def dequantize(self, t, q, n):
        out = np.zeros(n, np.float32)
        assert self.lib.qwref_dequantize(t, _p(np.ascontiguousarray(q)), _p(out), n) == 0
        return out

    def vec_dot(self, t, n, xq, yq):
        s = np.zeros(1, np.float32)
        assert self.lib.qwref_vec_dot(t, n, _p(xq), _p(yq), _p(s)) == 0
        return s[0]

    def unary(self, op, a, b=None, param=0.0, n_threads=1):
        a = np.ascontiguousarray(a, np.float32)
        ne0 = a.shape[-1]
        ne1 = a.size // ne0
        bb = None if b is None else np.ascontiguousarray(b, np.float32)
        if op == 1:
            out = np.zeros(a.shape, np.int32)
        elif op == 4:
            out = np.zeros(ne1, np.float32)
        else:
            out = np.zeros(a.shape, np.float32)
        assert self.lib.qwref_unary(op, _p(a), _p(bb), ne0, ne1, param, _p(out), n_threads) == 0
        return out

    def mul_mat_id(self, t, K, N, n_as, w, b, ids, n_threads=4):
        b = np.ascontiguousarray(b, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        T, b_ne1, _ = b.shape
        k = ids.shape[1]
        dst = np.zeros((T, k, N), np.float32)
        assert self.lib.qwref_mul_mat_id(t, K, N, n_as, _p(w), b_ne1, T, _p(b), k, _p(ids), _p(dst),
                                         n_threads) == 0
        return dst

    def layer(self, lw: LayerWeights, T: int, rms_eps: float = -1.0, scale: float = 0.0, n_threads: int = 4):
        return RefLayer(self, lw, T, rms_eps, scale, n_threads)


class RefLayer:
    def __init__(self, ref: RefGGML, lw: LayerWeights, T, rms_eps, scale, n_threads):
        assert lw.slot_of is None, "the reference graph indexes experts directly"
        self.ref, self.lw, self.T = ref, lw, T
        self.h = ref.lib.qwref_layer_create(lw.H, lw.E, lw.k, lw.F, T, lw.type_gate, lw.type_up,
                                            lw.type_down, _p(lw.router), _p(lw.gate), _p(lw.up),
                                            _p(lw.down), scale, rms_eps, n_threads)
        assert self.h

    def __call__(self, x, n_threads=0):
        lw, T = self.lw, self.T
        H, k, F, E = lw.H, lw.k, lw.F, lw.E
        x = np.ascontiguousarray(x, np.float32).reshape(T, H)
        r = dict(out=np.zeros((T, H), np.float32), xnext=np.zeros((T, H), np.float32),
                 ids=np.zeros((T, k), np.int32), weights=np.zeros((T, k), np.float32),
                 logits=np.zeros((T, E), np.float32), probs=np.zeros((T, E), np.float32),
                 gate=np.zeros((T, k, F), np.float32), up=np.zeros((T, k, F), np.float32),
                 act=np.zeros((T, k, F), np.float32), experts=np.zeros((T, k, H), np.float32))
        rc = self.ref.lib.qwref_layer_eval(self.h, _p(x), _p(r["out"]), _p(r["xnext"]), _p(r["ids"]),
                                           _p(r["weights"]), _p(r["logits"]), _p(r["probs"]), _p(r["gate"]),
                                           _p(r["up"]), _p(r["act"]), _p(r["experts"]), n_threads)
        assert rc == 0
        return r

    def __del__(self):
        try:
            self.ref.lib.qwref_layer_free(self.h)
        except Exception:
            pass


def have_ref() -> bool:
    return REF_SO.exists()


def have_ref_avx512() -> bool:
    """The AVX-512 reference build exists and this host has every ISA extension
    its flags enable (ggml's AVX-512 branch runs; elsewhere it would SIGILL)."""
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    need = ("avx512f", "avx512cd", "avx512vl", "avx512dq", "avx512bw", "avx512vbmi", "avx512_vnni", "avx512_bf16",
            "avx_vnni")
    return REF_SO_AVX512.exists() and all(f" {f}" in flags for f in need)
