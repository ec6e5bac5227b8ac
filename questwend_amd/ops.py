"""torch-facing wrappers over libqwmoe (device memory and streams come from torch).

Names follow the ggml ops they replace (ggml_mul_mat_id, ggml_soft_max +
argsort_top_k as ``router_topk``, ggml_swiglu_split, ggml_rms_norm).  Every call
goes through the C ABI; there is no CPU path.
"""
from __future__ import annotations

import ctypes as C

from . import BLOCK, Q8_0, Q8_K, Layer, check, lib, row_size, vec_dot_type


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


def mul_mat_id(qtype: int, w, K: int, N: int, n_as: int, b, ids, slot_of=None, out=None):
    """ggml_mul_mat_id.  w: uint8 with n_as matrices of N rows (dense);
    b: f32 [T, ne11, K]; ids: i32 [T, n_ids] (row stride may exceed n_ids);
    returns f32 [T, n_ids, N]."""
    torch = _torch()
    T, ne11, _ = b.shape
    n_ids = ids.shape[1]
    rs = row_size(qtype, K)
    if out is None:
        out = torch.empty((T, n_ids, N), dtype=torch.float32, device=b.device)
    n_slot_of = 0 if slot_of is None else slot_of.numel()
    check(lib().qwmoe_mul_mat_id(stream(), qtype, _ptr(w), K, N, n_as, rs, rs * N, _ptr(b), ne11, T,
                                 b.stride(1) * 4, b.stride(0) * 4, _ptr(ids), n_ids, ids.stride(0) * 4,
                                 _ptr(slot_of), n_slot_of, _ptr(out), out.stride(1) * 4, out.stride(0) * 4),
          "mul_mat_id")
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


def rms_norm(x, eps: float):
    torch = _torch()
    n = x.shape[-1]
    out = torch.empty_like(x)
    check(lib().qwmoe_rms_norm(stream(), _ptr(x), _ptr(out), n, x.numel() // n, eps), "rms_norm")
    return out


def make_layer(H, E, k, F, router, gate, up, down, types, n_slots=None, slots=None, scale=0.0) -> Layer:
    """Builds a ``qwmoe_layer`` from device tensors (dense expert matrices)."""
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
    return L


class DecodeStack:
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

    def status(self, clear: bool = True) -> int:
        v = C.c_int32(0)
        check(lib().qwmoe_decode_stack_status(stream(), self.h, C.byref(v), int(clear)), "decode_stack_status")
        return v.value

    def close(self) -> None:
        if self.h:
            lib().qwmoe_decode_stack_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


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
