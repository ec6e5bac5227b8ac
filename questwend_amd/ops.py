"""torch-facing wrappers over libqwmoe (device memory and streams come from torch).

Names follow the ggml ops they replace (ggml_mul_mat_id, ggml_soft_max +
argsort_top_k as ``router_topk``, ggml_swiglu_split, ggml_rms_norm).  Every call
goes through the C ABI; there is no CPU path.
"""
from __future__ import annotations

import atexit
import ctypes as C
import sys
import weakref

from . import (BLOCK, CACHE_COPY_ENGINE, CACHE_DRY_RUN, Q8_0, Q8_K, ExpertCacheConfig, ExpertCacheStats, ExpertSrc, GgufTensorInfo, Layer, SharedExpert,
               MoeHparams, check, lib, row_size, vec_dot_type)


def _torch():
    import torch  # noqa: WPS433
    return torch


def stream() -> int:
    return _torch().cuda.current_stream().cuda_stream


def init(device: int = 0, workspace_bytes: int = 0) -> None:
    check(lib().qwmoe_init(device, workspace_bytes), "qwmoe_init")


def shutdown() -> None:
    check(lib().qwmoe_shutdown(), "qwmoe_shutdown")


def set_mfma_min_rows(rows: int) -> int:
    """Experts with at least ``rows`` routed rows use the int8 matrix-core
    kernel (0: never; every output bit-exact).  Returns the previous value."""
    prev = lib().qwmoe_get_mfma_min_rows()
    check(lib().qwmoe_set_mfma_min_rows(rows), "set_mfma_min_rows")
    return prev


MFMA_BLOCK_SUM, MFMA_EXACT, MFMA_AUTO = 0, 1, 2


def set_mfma_form(form: int) -> int:
    """The matrix-core kernel's float tail: MFMA_EXACT replays ggml's fp32 lane
    chains (bit-identical), MFMA_BLOCK_SUM adds exact integer block sums in one
    fp32 chain per output, MFMA_AUTO is exact except for the down projections
    of the layer entry points.  The default is MFMA_EXACT; the other two are
    opt-in speed settings whose outputs drift from ggml's in the last bits.
    Returns the previous setting."""
    prev = int(lib().qwmoe_get_mfma_form())
    check(lib().qwmoe_set_mfma_form(int(form)), "set_mfma_form")
    return prev


def device_status(clear: bool = True) -> int:
    v = C.c_int32(0)
    check(lib().qwmoe_device_status(stream(), C.byref(v), int(clear)), "qwmoe_device_status")
    return v.value


def _ptr(t):
    return None if t is None else t.data_ptr()


def quantize_act(vdt: int, x):
    """x: f32 [..., K] (rows dense or row-strided) -> uint8 [rows, row_size(vdt, K)]."""
    torch = _torch()
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    out = torch.empty((x2.shape[0], row_size(vdt, K)), dtype=torch.uint8, device=x.device)
    check(lib().qwmoe_quantize_act(stream(), vdt, _ptr(x2), K, x2.shape[0], 1, x2.stride(0) * 4,
                                   x2.stride(0) * 4 * x2.shape[0], _ptr(out)), "quantize_act")
    return out


def quantize_chunk(qtype: int, x):
    """ggml_quantize_chunk: f32 [nrows, n_per_row] -> uint8 [nrows, row_size]."""
    torch = _torch()
    n_per_row = x.shape[-1]
    x2 = x.reshape(-1, n_per_row).contiguous()
    out = torch.empty((x2.shape[0], row_size(qtype, n_per_row)), dtype=torch.uint8, device=x.device)
    check(lib().qwmoe_quantize_chunk(stream(), qtype, _ptr(x2), _ptr(out), x2.shape[0], n_per_row), "quantize_chunk")
    return out


def quantize_chunk_into(qtype: int, x, out) -> None:
    n_per_row = x.shape[-1]
    check(lib().qwmoe_quantize_chunk(stream(), qtype, _ptr(x), _ptr(out), x.numel() // n_per_row, n_per_row),
          "quantize_chunk")


def dequantize(qtype: int, q, n: int):
    torch = _torch()
    out = torch.empty(n, dtype=torch.float32, device=q.device)
    check(lib().qwmoe_dequantize(stream(), qtype, _ptr(q), _ptr(out), n), "dequantize")
    return out


def randn_(t, seed: int, mean: float = 0.0, std: float = 1.0):
    check(lib().qwmoe_fill_randn(stream(), _ptr(t), t.numel(), seed, mean, std), "fill_randn")
    return t


def mul_mat_id(qtype: int, w, K: int, N: int, n_as: int, b, ids, slot_of=None, out=None, noalloc=False):
    """ggml_mul_mat_id.  w: uint8 with n_as matrices of N rows (dense);
    b: f32 [T, ne11, K]; ids: i32 [T, n_ids] (row stride may exceed n_ids);
    returns f32 [T, n_ids, N].  noalloc: through qwmoe_mul_mat_id_noalloc
    (static scratch, no library workspace)."""
    torch = _torch()
    T, ne11, _ = b.shape
    n_ids = ids.shape[1]
    rs = row_size(qtype, K)
    if out is None:
        out = torch.empty((T, n_ids, N), dtype=torch.float32, device=b.device)
    n_slot_of = 0 if slot_of is None else slot_of.numel()
    fn = lib().qwmoe_mul_mat_id_noalloc if noalloc else lib().qwmoe_mul_mat_id
    check(fn(stream(), qtype, _ptr(w), K, N, n_as, rs, rs * N, _ptr(b), ne11, T, b.stride(1) * 4, b.stride(0) * 4,
             _ptr(ids), n_ids, ids.stride(0) * 4, _ptr(slot_of), n_slot_of, _ptr(out), out.stride(1) * 4,
             out.stride(0) * 4),
          "mul_mat_id_noalloc" if noalloc else "mul_mat_id")
    return out


def group_by_expert(ids, n_as: int):
    torch = _torch()
    T, n_ids = ids.shape
    dev = ids.device
    counts = torch.empty(n_as, dtype=torch.int32, device=dev)
    offsets = torch.empty(n_as + 1, dtype=torch.int32, device=dev)
    rows = torch.empty((T * n_ids, 2), dtype=torch.int32, device=dev)
    check(lib().qwmoe_group_by_expert(stream(), _ptr(ids), n_ids, T, ids.stride(0) * 4, n_as, _ptr(counts),
                                      _ptr(offsets), _ptr(rows)), "group_by_expert")
    return counts, offsets, rows


def router_topk(W, x, k: int, clamp_min: float = 6.103515625e-5, scale: float = 0.0, want_probs: bool = False):
    """W: f32 [E, H]; x: f32 [T, H] -> ids i32 [T, k], weights f32 [T, k] (, probs [T, E])."""
    torch = _torch()
    E, H = W.shape
    T = x.shape[0]
    ids = torch.empty((T, k), dtype=torch.int32, device=x.device)
    w = torch.empty((T, k), dtype=torch.float32, device=x.device)
    probs = torch.empty((T, E), dtype=torch.float32, device=x.device) if want_probs else None
    check(lib().qwmoe_router_topk(stream(), _ptr(W), _ptr(x), H, E, k, T, x.stride(0) * 4, clamp_min, scale,
                                  _ptr(ids), _ptr(w), _ptr(probs)), "router_topk")
    return (ids, w, probs) if want_probs else (ids, w)


def plan_slices(sel, n_expert: int, cap: int, max_slice: int = 1024):
    """plan_slices (core/runtime.cpp:2144-2170) on the host: sel int32 [T, n_used]
    -> ([(t0, len)], union in first-use order)."""
    import numpy as np
    a = np.ascontiguousarray(sel, dtype=np.int32)
    T, n_used = a.shape
    out = np.zeros(2 * max(T, 1), np.int32)
    un = np.zeros(n_expert, np.int32)
    ns, nu = C.c_int(0), C.c_int(0)
    check(lib().qwmoe_plan_slices(a.ctypes.data, T, n_used, n_expert, cap, max_slice, out.ctypes.data, C.byref(ns),
                                  un.ctypes.data, C.byref(nu)), "plan_slices")
    return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(ns.value)], un[:nu.value].tolist()


def router_topk_resident(W, x, k: int, mask=None, want: bool = True, clamp_min: float = 6.103515625e-5,
                         scale: float = 0.0):
    """Resident-only routing: mask f32 [E] (0 / -inf) added to the logits before
    the softmax; want = the unmasked top k.  Returns ids, weights (, want) [T, k]."""
    torch = _torch()
    E, H = W.shape
    T = x.shape[0]
    ids = torch.empty((T, k), dtype=torch.int32, device=x.device)
    w = torch.empty((T, k), dtype=torch.float32, device=x.device)
    wt = torch.empty((T, k), dtype=torch.int32, device=x.device) if want else None
    check(lib().qwmoe_router_topk_resident(stream(), _ptr(W), _ptr(x), H, E, k, T, x.stride(0) * 4, clamp_min, scale,
                                           _ptr(mask), _ptr(wt), _ptr(ids), _ptr(w), None), "router_topk_resident")
    return (ids, w, wt) if want else (ids, w)


def swiglu(gate, up):
    torch = _torch()
    n = gate.shape[-1]
    out = torch.empty_like(gate)
    check(lib().qwmoe_swiglu(stream(), _ptr(gate), _ptr(up), _ptr(out), n, gate.numel() // n), "swiglu")
    return out


def weighted_sum(experts, weights):
    """experts: f32 [T, k, H]; weights: [T, k] -> [T, H]."""
    torch = _torch()
    T, k, H = experts.shape
    out = torch.empty((T, H), dtype=torch.float32, device=experts.device)
    check(lib().qwmoe_weighted_sum(stream(), _ptr(experts), _ptr(weights), _ptr(out), H, k, T), "weighted_sum")
    return out


def rms_norm(x, eps: float, weight=None):
    """ggml_rms_norm of each row of x; with ``weight`` [n], then ggml_mul by it
    (the router input of a decoder layer)."""
    torch = _torch()
    n = x.shape[-1]
    out = torch.empty_like(x)
    if weight is None:
        check(lib().qwmoe_rms_norm(stream(), _ptr(x), _ptr(out), n, x.numel() // n, eps), "rms_norm")
    else:
        check(lib().qwmoe_rms_norm_mul(stream(), _ptr(x), _ptr(weight), _ptr(out), n, x.numel() // n, eps),
              "rms_norm_mul")
    return out


def make_shared_expert(F: int, gate, up, down, gate_inp, types) -> SharedExpert:
    """A qwmoe_shared_expert over dense device tensors: gate / up [F, row(H)],
    down [H, row(F)] (uint8 rows), gate_inp f32 [H]."""
    return SharedExpert(F, types[0], types[1], types[2], _ptr(gate), _ptr(up), _ptr(down), gate.stride(0),
                        up.stride(0), down.stride(0), _ptr(gate_inp))


def shared_expert_add(se: SharedExpert, x, moe_out, resid=None, out=None):
    """moe_out + shared expert(x) (+ resid) for x, moe_out, resid f32 [T, H]."""
    T, H = x.shape
    if out is None:
        out = _torch().empty_like(moe_out)
    check(lib().qwmoe_shared_expert_add(stream(), C.byref(se), H, _ptr(x), T, _ptr(moe_out), _ptr(resid), _ptr(out)),
          "shared_expert_add")
    return out


def make_layer(H, E, k, F, router, gate, up, down, types, n_slots=None, slots=None, scale=0.0, resmask=None,
               want_ids=None) -> Layer:
    """Builds a ``qwmoe_layer`` from device tensors (dense expert matrices).
    resmask: f32 [E] (0 / -inf) for resident-only routing; want_ids: i32 [T, k]
    receiving the unmasked top k (both optional; the caller keeps them alive)."""
    tg, tu, td = types
    rg, ru, rd = row_size(tg, H), row_size(tu, H), row_size(td, F)
    ns = n_slots or (E, E, E)
    sg, su, sd = slots if slots is not None else (None, None, None)
    L = Layer()
    L.n_embd, L.n_expert, L.n_expert_used, L.n_ff = H, E, k, F
    L.expert_weights_scale = scale
    L.router = _ptr(router)
    L.type_gate, L.type_up, L.type_down = tg, tu, td
    L.gate, L.up, L.down = _ptr(gate), _ptr(up), _ptr(down)
    L.gate_nb1, L.gate_nb2 = rg, rg * F
    L.up_nb1, L.up_nb2 = ru, ru * F
    L.down_nb1, L.down_nb2 = rd, rd * H
    L.n_slots_gate, L.n_slots_up, L.n_slots_down = ns
    L.slot_gate, L.slot_up, L.slot_down = _ptr(sg), _ptr(su), _ptr(sd)
    L.resmask, L.want_ids = _ptr(resmask), _ptr(want_ids)
    return L


# Handles (decode / layer stacks, expert caches, GGUF files) still open when
# the program ends are freed by an atexit hook: Python runs it before the
# interpreter shuts down and before the shared libraries' static destructors
# (the HIP runtime's among them), so hipFree / hipHostFree, stream
# synchronisation and worker-thread joins run against a runtime that is whole.
# A finaliser that runs during interpreter shutdown does nothing: the process
# is ending and its memory goes with it.
_open_handles: "weakref.WeakSet" = weakref.WeakSet()


@atexit.register
def _close_open_handles() -> None:
    for obj in list(_open_handles):
        try:
            obj.close()
        except Exception:  # noqa: BLE001  (best effort at exit)
            pass


class _Handle:
    h = None

    def _opened(self) -> None:
        _open_handles.add(self)

    def close(self) -> None:   # each handle class frees its object in _free()
        if self.h:
            self._free()
            self.h = None
        _open_handles.discard(self)

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass


class DecodeStack(_Handle):
    """A persistent-kernel decode stack over ``layers`` (qwmoe_decode_stack_*).

    Keeps references to the layer tensors it points at; ``run`` pushes one
    token through every layer in a single launch."""

    def __init__(self, layers: list[Layer], rms_eps: float = 1e-6, keepalive=None):
        arr = (Layer * len(layers))(*layers)
        h = C.c_void_p()
        check(lib().qwmoe_decode_stack_create(C.cast(arr, C.c_void_p), len(layers), rms_eps, C.byref(h)),
              "decode_stack_create")
        self.h, self.n_layer, self._keep = h, len(layers), (arr, keepalive)
        self.H, self.k = layers[0].n_embd, layers[0].n_expert_used
        self._opened()

    def run(self, x, out, x_out=None, ids=None, weights=None) -> None:
        check(lib().qwmoe_decode_stack_run(stream(), self.h, _ptr(x), _ptr(out), _ptr(x_out), _ptr(ids),
                                           _ptr(weights)), "decode_stack_run")

    def __call__(self, x, want_ids: bool = True):
        torch = _torch()
        out = torch.empty(self.H, dtype=torch.float32, device=x.device)
        xo = torch.empty(self.H, dtype=torch.float32, device=x.device)
        ids = torch.empty((self.n_layer, self.k), dtype=torch.int32, device=x.device) if want_ids else None
        w = torch.empty((self.n_layer, self.k), dtype=torch.float32, device=x.device) if want_ids else None
        self.run(x, out, xo, ids, w)
        return out, xo, ids, w

    def kernel(self) -> int:
        """1: one workgroup per CU; 2: one expert per XCD; 3: the same, device-scope words;
        4, 5: the forms of 2, 3 for wide layers (H = 4096, F = 1536)."""
        return int(lib().qwmoe_decode_stack_kernel(self.h))

    def status(self, clear: bool = True) -> int:
        v = C.c_int32(0)
        check(lib().qwmoe_decode_stack_status(stream(), self.h, C.byref(v), int(clear)), "decode_stack_status")
        return v.value

    def _free(self) -> None:
        lib().qwmoe_decode_stack_free(self.h)


class LayerStack(_Handle):
    """T-token batches through a stack of MoE FFN layers (qwmoe_layer_stack_*):
    the verify forward's FFN half, one captured HIP graph per T."""

    def __init__(self, layers: list[Layer], rms_eps: float = 1e-6, max_tokens: int = 8, graphs: bool = True,
                 keepalive=None):
        arr = (Layer * len(layers))(*layers)
        h = C.c_void_p()
        check(lib().qwmoe_layer_stack_create(C.cast(arr, C.c_void_p), len(layers), rms_eps, max_tokens,
                                             0 if graphs else 1, C.byref(h)), "layer_stack_create")
        self.h, self.n_layer, self._keep = h, len(layers), (arr, keepalive)
        self.H, self.k = layers[0].n_embd, layers[0].n_expert_used
        self._opened()

    def __call__(self, x, want_ids: bool = True):
        """x: f32 [T, H] -> (out [T, H], x_out [T, H], ids [n_layer, T, k], weights)."""
        torch = _torch()
        T = x.shape[0]
        out = torch.empty((T, self.H), dtype=torch.float32, device=x.device)
        xo = torch.empty_like(out)
        ids = torch.empty((self.n_layer, T, self.k), dtype=torch.int32, device=x.device) if want_ids else None
        w = torch.empty((self.n_layer, T, self.k), dtype=torch.float32, device=x.device) if want_ids else None
        check(lib().qwmoe_layer_stack_run(stream(), self.h, _ptr(x), T, _ptr(out), _ptr(xo), _ptr(ids), _ptr(w)),
              "layer_stack_run")
        return out, xo, ids, w

    def captures(self) -> int:
        return lib().qwmoe_layer_stack_captures(self.h)

    def kernel(self) -> int:
        """1: the per-layer chain; 2: one persistent launch for 2 <= T <= 8 (3: device-scope words)."""
        return int(lib().qwmoe_layer_stack_kernel(self.h))

    def kernel_t1(self) -> int:
        """The decode kernel a T = 1 run takes (qwmoe_decode_stack_kernel's value), 0 for the chain."""
        return int(lib().qwmoe_layer_stack_kernel_t1(self.h))

    def status(self, clear: bool = True) -> int:
        v = C.c_int32(0)
        check(lib().qwmoe_layer_stack_status(stream(), self.h, C.byref(v), int(clear)), "layer_stack_status")
        return v.value

    def _free(self) -> None:
        lib().qwmoe_layer_stack_free(self.h)


def ffn_layer(layer: Layer, x, rms_eps: float = -1.0):
    """One MoE FFN layer.  x: f32 [T, H] -> (out, x_next or None, ids, weights)."""
    torch = _torch()
    T, H = x.shape
    k = layer.n_expert_used
    out = torch.empty((T, H), dtype=torch.float32, device=x.device)
    xn = torch.empty((T, H), dtype=torch.float32, device=x.device) if rms_eps >= 0 else None
    ids = torch.empty((T, k), dtype=torch.int32, device=x.device)
    w = torch.empty((T, k), dtype=torch.float32, device=x.device)
    check(lib().qwmoe_ffn_layer(stream(), C.byref(layer), _ptr(x), T, _ptr(out), rms_eps, _ptr(xn), _ptr(ids),
                                _ptr(w)), "ffn_layer")
    return out, xn, ids, w


def make_attn_layer(H, n_head, n_head_kv, D, attn_norm, wq, wk, wv, wo, types, q_norm, k_norm, ffn_norm,
                    k_cache, v_cache, rope_freq_base=1e6):
    """Builds a ``qwmoe_attn_layer`` from device tensors (dense weight rows, f16
    caches [n_ctx, n_head_kv * D] as int16/float16 tensors; the caller keeps
    them alive).  types: (q, k, v, o) ggml type ids."""
    from . import AttnLayer
    tq, tk, tv, to = types
    L = AttnLayer()
    L.n_embd, L.n_head, L.n_head_kv, L.n_embd_head, L.n_rot = H, n_head, n_head_kv, D, D
    L.rope_freq_base = rope_freq_base
    L.attn_norm = _ptr(attn_norm)
    L.type_q, L.type_k, L.type_v, L.type_o = tq, tk, tv, to
    L.wq, L.wq_nb1 = _ptr(wq), row_size(tq, H)
    L.wk, L.wk_nb1 = _ptr(wk), row_size(tk, H)
    L.wv, L.wv_nb1 = _ptr(wv), row_size(tv, H)
    L.wo, L.wo_nb1 = _ptr(wo), row_size(to, n_head * D)
    L.q_norm, L.k_norm, L.ffn_norm = _ptr(q_norm), _ptr(k_norm), _ptr(ffn_norm)
    L.k_cache, L.v_cache = _ptr(k_cache), _ptr(v_cache)
    L.n_ctx = k_cache.shape[0]
    return L


def attn_seg(layer, h, n_past: int, rms_eps: float = 1e-6, want_ffn_in: bool = True):
    """The attention half of Seg A for h f32 [T, H] at positions n_past ..:
    (attn_resid, ffn_in or None); the layer's caches get rows n_past .. n_past + T - 1."""
    torch = _torch()
    T, H = h.shape
    resid = torch.empty((T, H), dtype=torch.float32, device=h.device)
    fin = torch.empty((T, H), dtype=torch.float32, device=h.device) if want_ffn_in else None
    check(lib().qwmoe_attn_seg(stream(), C.byref(layer), _ptr(h), T, n_past, rms_eps, _ptr(resid), _ptr(fin)),
          "attn_seg")
    return resid, fin


def make_gdn_layer(H, S, H_k, H_v, d_conv, types, attn_norm, w_qkv, w_gate, w_beta, w_alpha, w_out, dt_bias, ssm_a,
                   conv1d, ssm_norm, ffn_norm, conv_state, ssm_state):
    """Builds a ``qwmoe_gdn_layer`` from device tensors (dense weight rows; f32
    conv1d [conv_ch, d_conv], conv_state [conv_ch, d_conv - 1], ssm_state
    [H_v, S, S]; the caller keeps them alive).  types: (qkv, gate, beta, alpha,
    out) ggml type ids."""
    from . import GdnLayer
    L = GdnLayer()
    L.n_embd, L.d_state, L.n_group, L.dt_rank, L.d_conv = H, S, H_k, H_v, d_conv
    L.attn_norm = _ptr(attn_norm)
    L.type_qkv, L.type_gate, L.type_beta, L.type_alpha, L.type_out = types
    L.w_qkv, L.w_qkv_nb1 = _ptr(w_qkv), row_size(types[0], H)
    L.w_gate, L.w_gate_nb1 = _ptr(w_gate), row_size(types[1], H)
    L.w_beta, L.w_beta_nb1 = _ptr(w_beta), row_size(types[2], H)
    L.w_alpha, L.w_alpha_nb1 = _ptr(w_alpha), row_size(types[3], H)
    L.w_out, L.w_out_nb1 = _ptr(w_out), row_size(types[4], H_v * S)
    L.dt_bias, L.ssm_a, L.conv1d, L.ssm_norm, L.ffn_norm = (_ptr(dt_bias), _ptr(ssm_a), _ptr(conv1d),
                                                             _ptr(ssm_norm), _ptr(ffn_norm))
    L.conv_state, L.ssm_state = _ptr(conv_state), _ptr(ssm_state)
    return L


def gdn_seg(layer, h, rms_eps: float = 1e-6, want_ffn_in: bool = True):
    """The gated-delta-net half of Seg A for h f32 [T, H]: (attn_resid, ffn_in or
    None); the layer's conv and recurrent states advance by T tokens."""
    torch = _torch()
    T, H = h.shape
    resid = torch.empty((T, H), dtype=torch.float32, device=h.device)
    fin = torch.empty((T, H), dtype=torch.float32, device=h.device) if want_ffn_in else None
    check(lib().qwmoe_gdn_seg(stream(), C.byref(layer), _ptr(h), T, rms_eps, _ptr(resid), _ptr(fin)), "gdn_seg")
    return resid, fin


def decoder_layer(attn, moe: Layer, h, n_past: int, rms_eps: float = 1e-6):
    """A whole Qwen3-MoE decoder layer for h f32 [T, H]: (h_out, ids, weights)."""
    torch = _torch()
    T, H = h.shape
    k = moe.n_expert_used
    out = torch.empty((T, H), dtype=torch.float32, device=h.device)
    ids = torch.empty((T, k), dtype=torch.int32, device=h.device)
    w = torch.empty((T, k), dtype=torch.float32, device=h.device)
    check(lib().qwmoe_decoder_layer(stream(), C.byref(attn), C.byref(moe), _ptr(h), T, n_past, rms_eps, _ptr(out),
                                    _ptr(ids), _ptr(w)), "decoder_layer")
    return out, ids, w


class Gguf(_Handle):
    """A GGUF model file (or shard set) opened through qwmoe_gguf_*: metadata on
    the host, MoE layers loaded into device memory on request."""

    _SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}

    def __init__(self, path):
        h = C.c_void_p()
        check(lib().qwmoe_gguf_open(str(path).encode(), C.byref(h)), "gguf_open")
        self.h = h
        self._opened()

    def _free(self) -> None:
        lib().qwmoe_gguf_close(self.h)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def shards(self) -> list[dict]:
        out = []
        for i in range(lib().qwmoe_gguf_n_shards(self.h)):
            v, a, d = C.c_uint32(), C.c_uint64(), C.c_uint64()
            check(lib().qwmoe_gguf_shard_info(self.h, i, C.byref(v), C.byref(a), C.byref(d)), "gguf_shard_info")
            out.append({"version": v.value, "alignment": a.value, "data_offset": d.value})
        return out

    def kv(self) -> list[dict]:
        import struct
        out = []
        for i in range(lib().qwmoe_gguf_n_kv(self.h)):
            key, t, at, n, data = C.c_char_p(), C.c_int32(), C.c_int32(), C.c_uint64(), C.c_void_p()
            check(lib().qwmoe_gguf_kv(self.h, i, C.byref(key), C.byref(t), C.byref(at), C.byref(n), C.byref(data)),
                  "gguf_kv")
            e = {"key": key.value.decode(), "type": t.value}
            et = at.value if t.value == 9 else t.value
            if t.value == 9:
                e.update(arr_type=at.value, n=n.value)
            if et == 8:
                vals = []
                for j in range(n.value):
                    s = C.c_char_p()
                    check(lib().qwmoe_gguf_kv_str(self.h, i, j, C.byref(s)), "gguf_kv_str")
                    vals.append(s.value.decode())
            else:
                f = self._SCALAR[et]
                sz = struct.calcsize("<" + f)
                raw = C.string_at(data.value, n.value * sz) if n.value else b""
                vals = list(struct.unpack(f"<{n.value}{f}", raw))
            e["value"] = vals if t.value == 9 else vals[0]
            out.append(e)
        return out

    def tensors(self) -> list[dict]:
        out = []
        for i in range(lib().qwmoe_gguf_n_tensors(self.h)):
            ti = GgufTensorInfo()
            check(lib().qwmoe_gguf_tensor_at(self.h, i, C.byref(ti)), "gguf_tensor_at")
            out.append(self._info(ti))
        return out

    def tensor(self, name: str):
        ti = GgufTensorInfo()
        idx = lib().qwmoe_gguf_find_tensor(self.h, name.encode(), C.byref(ti))
        return None if idx < 0 else self._info(ti)

    @staticmethod
    def _info(ti) -> dict:
        return {"name": ti.name.decode(), "type": ti.type, "n_dims": ti.n_dims, "ne": list(ti.ne),
                "offset": ti.offset, "file_offset": ti.file_offset, "size": ti.nbytes, "shard": ti.shard}

    def get_u32(self, key: str, default: int = 0) -> int:
        v = C.c_uint32()
        check(lib().qwmoe_gguf_get_u32(self.h, key.encode(), default, C.byref(v)), "gguf_get_u32")
        return v.value

    def get_f32(self, key: str, default: float = 0.0) -> float:
        v = C.c_float()
        check(lib().qwmoe_gguf_get_f32(self.h, key.encode(), default, C.byref(v)), "gguf_get_f32")
        return v.value

    def get_str(self, key: str, default: str = ""):
        v = C.c_char_p()
        check(lib().qwmoe_gguf_get_str(self.h, key.encode(), default.encode(), C.byref(v)), "gguf_get_str")
        return v.value.decode()

    def hparams(self) -> dict:
        hp = MoeHparams()
        check(lib().qwmoe_gguf_moe_hparams(self.h, C.byref(hp)), "gguf_moe_hparams")
        return {"arch": hp.arch.decode(), "n_layer": hp.n_layer, "n_embd": hp.n_embd, "n_expert": hp.n_expert,
                "n_expert_used": hp.n_expert_used, "n_ff_exp": hp.n_ff_exp,
                "expert_weights_scale": hp.expert_weights_scale}

    def layer_bytes(self, il: int) -> int:
        n = C.c_size_t()
        check(lib().qwmoe_gguf_moe_layer_bytes(self.h, il, C.byref(n)), "gguf_moe_layer_bytes")
        return n.value

    def load_layer(self, il: int, device="cuda:0"):
        """Layer il's router and experts in a new device buffer -> (Layer, buffer)."""
        torch = _torch()
        buf = torch.empty(self.layer_bytes(il), dtype=torch.uint8, device=device)
        L = Layer()
        check(lib().qwmoe_gguf_load_moe_layer(stream(), self.h, il, _ptr(buf), buf.numel(), C.byref(L)),
              "gguf_load_moe_layer")
        return L, buf


class ExpertCache(_Handle):
    """Expert slot pools in device memory fed from host memory or a file,
    through qwmoe_expert_cache_* (ExpertCache, core/expert_cache.h:39-166).

    Construct with ``sources`` = [role][layer] dicts {type, ne0, ne1, host (an
    address) or path + file_offset}, or with ``ExpertCache.from_gguf``.  Every
    copy goes on ``stream`` (torch's current stream by default); a dry run keeps
    the bookkeeping only."""

    ROLES = ("gate", "up", "down")

    def __init__(self, n_layer: int, n_expert: int, sources, vram_budget: int, n_used: int, io_threads: int = 0,
                 dry_run: bool = False, stream_handle=None, copy_engine: bool = False, _handle=None):
        self.n_layer, self.n_expert = n_layer, n_expert
        self._keep = []
        if _handle is not None:
            self.h = _handle
            self._opened()
            return
        arr = (ExpertSrc * (3 * n_layer))()
        for r in range(3):
            for il in range(n_layer):
                s = sources[r][il]
                e = arr[r * n_layer + il]
                e.type, e.ne0, e.ne1 = s["type"], s["ne0"], s["ne1"]
                e.host = s.get("host")
                if s.get("path") is not None:
                    b = str(s["path"]).encode()
                    self._keep.append(b)
                    e.path = b
                    e.file_offset = s.get("file_offset", 0)
        flags = (CACHE_DRY_RUN if dry_run else 0) | (CACHE_COPY_ENGINE if copy_engine else 0)
        cfg = ExpertCacheConfig(vram_budget, n_used, io_threads, flags)
        h = C.c_void_p()
        st = None if dry_run else (stream_handle if stream_handle is not None else stream())
        check(lib().qwmoe_expert_cache_create(st, n_layer, n_expert, arr, C.byref(cfg), C.byref(h)),
              "expert_cache_create")
        self.h = h
        self._opened()

    @classmethod
    def from_gguf(cls, g: "Gguf", tier: int, vram_budget: int, n_used: int = 0, io_threads: int = 0,
                  dry_run: bool = False, stream_handle=None):
        cfg = ExpertCacheConfig(vram_budget, n_used, io_threads, CACHE_DRY_RUN if dry_run else 0)
        h = C.c_void_p()
        st = None if dry_run else (stream_handle if stream_handle is not None else stream())
        check(lib().qwmoe_expert_cache_create_gguf(st, g.h, tier, C.byref(cfg), C.byref(h)), "expert_cache_create_gguf")
        hp = g.hparams()
        return cls(hp["n_layer"], hp["n_expert"], None, 0, 0, _handle=h)

    def _free(self) -> None:
        lib().qwmoe_expert_cache_free(self.h)

    def pools(self) -> list[dict]:
        out = []
        for i in range(lib().qwmoe_expert_cache_n_pools(self.h)):
            role, t, ne0, ne1, ns, slab, base = (C.c_int32(), C.c_int32(), C.c_int64(), C.c_int64(), C.c_int64(),
                                                 C.c_uint64(), C.c_void_p())
            check(lib().qwmoe_expert_cache_pool_info(self.h, i, C.byref(role), C.byref(t), C.byref(ne0), C.byref(ne1),
                                                     C.byref(ns), C.byref(slab), C.byref(base)), "pool_info")
            out.append({"role": role.value, "type": t.value, "ne0": ne0.value, "ne1": ne1.value,
                        "n_slots": ns.value, "slab": slab.value, "base": base.value})
        return out

    def pool_of(self, role: int, layer: int) -> int:
        r = lib().qwmoe_expert_cache_pool_of(self.h, role, layer)
        check(min(r, 0), "pool_of")
        return r

    def min_slots(self) -> int:
        return lib().qwmoe_expert_cache_min_slots(self.h)

    def capacity(self, layer: int) -> int:
        r = lib().qwmoe_expert_cache_capacity(self.h, layer)
        check(min(r, 0), "capacity")
        return r

    def ensure(self, layer: int, ids) -> tuple[list[int], list[int], list[int]]:
        n = len(ids)
        a = (C.c_int32 * max(n, 1))(*ids)
        g, u, d = ((C.c_int32 * max(n, 1))() for _ in range(3))
        check(lib().qwmoe_expert_cache_ensure(self.h, layer, a, n, g, u, d), "expert_cache_ensure")
        return list(g[:n]), list(u[:n]), list(d[:n])

    def ensure_resident(self, layer: int, expert: int) -> None:
        check(lib().qwmoe_expert_cache_ensure_resident(self.h, layer, expert), "expert_cache_ensure_resident")

    def touch(self, role: int, layer: int, expert: int) -> None:
        check(lib().qwmoe_expert_cache_touch(self.h, role, layer, expert), "expert_cache_touch")

    def resident(self, role: int, layer: int, expert: int) -> bool:
        r = lib().qwmoe_expert_cache_resident(self.h, role, layer, expert)
        check(min(r, 0), "expert_cache_resident")
        return r == 1

    def verify(self, ids, touch: bool = True) -> int:
        """ids: int32 [n_layer, k] (host array or tensor) -> entries missing in any role."""
        import numpy as np
        a = np.ascontiguousarray(ids.cpu().numpy() if hasattr(ids, "cpu") else ids, dtype=np.int32)
        r = lib().qwmoe_expert_cache_verify(self.h, a.ctypes.data, a.shape[0], a.shape[1], int(touch))
        check(min(r, 0), "expert_cache_verify")
        return r

    def resmask(self, floor_res: int, device_out=None):
        """The resident-decode mask [n_layer, n_expert] (0 / -inf) as a numpy array
        and whether every layer is masked; device_out (f32 tensor of that shape)
        receives a copy on the cache's stream."""
        import numpy as np
        m = np.zeros((self.n_layer, self.n_expert), np.float32)
        r = lib().qwmoe_expert_cache_resmask(self.h, floor_res, m.ctypes.data, _ptr(device_out))
        check(min(r, 0), "expert_cache_resmask")
        return m, r == 1

    def refill(self, sel, want, budget: int, cursor: int) -> tuple[int, int]:
        """Background refill after a masked decode: sel / want int32 [n_layer, k]
        (host arrays or tensors).  Returns (fetched, next cursor)."""
        import numpy as np
        a = np.ascontiguousarray(sel.cpu().numpy() if hasattr(sel, "cpu") else sel, dtype=np.int32)
        b = np.ascontiguousarray(want.cpu().numpy() if hasattr(want, "cpu") else want, dtype=np.int32)
        cur = C.c_int(cursor)
        r = lib().qwmoe_expert_cache_refill(self.h, a.ctypes.data, b.ctypes.data, a.shape[0], a.shape[1], budget,
                                            C.byref(cur))
        check(min(r, 0), "expert_cache_refill")
        return r, cur.value

    def slot_of_row(self, role: int, layer: int) -> list[int]:
        p = lib().qwmoe_expert_cache_slot_of_row(self.h, role, layer)
        if not p:
            raise ValueError("role/layer out of range")
        return list((C.c_int32 * self.n_expert).from_address(p))

    def device_row(self, role: int, layer: int) -> int:
        return lib().qwmoe_expert_cache_device_row(self.h, role, layer) or 0

    def layer(self, layer: int, L: Layer | None = None) -> Layer:
        L = L if L is not None else Layer()
        check(lib().qwmoe_expert_cache_layer(self.h, layer, C.byref(L)), "expert_cache_layer")
        return L

    def stats(self) -> dict:
        s = ExpertCacheStats()
        check(lib().qwmoe_expert_cache_get_stats(self.h, C.byref(s)), "expert_cache_stats")
        return {"hits": s.hits, "misses": s.misses, "evictions": s.evictions, "fetch_ms": s.fetch_ms,
                "fetch_bytes": s.fetch_bytes}

    def save_profile(self, path) -> None:
        check(lib().qwmoe_expert_cache_save_profile(self.h, str(path).encode()), "expert_cache_save_profile")

    def load_prefetch(self, path) -> int:
        n = C.c_uint64()
        check(lib().qwmoe_expert_cache_load_prefetch(self.h, str(path).encode(), C.byref(n)), "expert_cache_load_prefetch")
        return n.value

    def sync(self) -> None:
        check(lib().qwmoe_expert_cache_sync(self.h), "expert_cache_sync")

    def run_layer(self, layer: int, L: Layer, x, rms_eps: float = -1.0):
        """decode_cached for one layer: router ids read back, ensure(), the layer on
        the pools.  x: f32 [T, H] -> (out, x_next or None, ids, weights)."""
        torch = _torch()
        T, H = x.shape
        k = L.n_expert_used
        out = torch.empty((T, H), dtype=torch.float32, device=x.device)
        xn = torch.empty((T, H), dtype=torch.float32, device=x.device) if rms_eps >= 0 else None
        ids = torch.empty((T, k), dtype=torch.int32, device=x.device)
        w = torch.empty((T, k), dtype=torch.float32, device=x.device)
        check(lib().qwmoe_expert_cache_run_layer(self.h, layer, C.byref(L), _ptr(x), T, _ptr(out), rms_eps, _ptr(xn),
                                                 _ptr(ids), _ptr(w)), "expert_cache_run_layer")
        return out, xn, ids, w

    def run_batch(self, layer: int, L: Layer, x, rms_eps: float = -1.0, max_slice: int = 1024):
        """The chunked prefill's layer through the cache: ids read back, planned
        into slices within the pools' capacity, ensure() + the layer per slice.
        x: f32 [T, H] -> (out, x_next or None, ids, weights, n_slices)."""
        torch = _torch()
        T, H = x.shape
        k = L.n_expert_used
        out = torch.empty((T, H), dtype=torch.float32, device=x.device)
        xn = torch.empty((T, H), dtype=torch.float32, device=x.device) if rms_eps >= 0 else None
        ids = torch.empty((T, k), dtype=torch.int32, device=x.device)
        w = torch.empty((T, k), dtype=torch.float32, device=x.device)
        ns = C.c_int(0)
        check(lib().qwmoe_expert_cache_run_batch(self.h, layer, C.byref(L), _ptr(x), T, _ptr(out), rms_eps, _ptr(xn),
                                                 _ptr(ids), _ptr(w), max_slice, C.byref(ns)), "expert_cache_run_batch")
        return out, xn, ids, w, ns.value

    def plan_slices(self, layer: int, sel, max_slice: int = 1024) -> list[tuple[int, int]]:
        import numpy as np
        a = np.ascontiguousarray(sel, dtype=np.int32)
        T = a.shape[0]
        out = np.zeros(2 * max(T, 1), np.int32)
        ns = C.c_int(0)
        check(lib().qwmoe_expert_cache_plan_slices(self.h, layer, a.ctypes.data, T, max_slice, out.ctypes.data,
                                                   C.byref(ns)), "expert_cache_plan_slices")
        return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(ns.value)]
