"""questwend_amd -- MI355X-native quantized MoE expert-FFN path for QuestWend.

The product is the C-ABI library ``libqwmoe.so`` (declared in include/qwmoe.h,
built from questwend_amd/csrc by ``questwend_amd.build``).  This module is a
thin ctypes binding over it for Python callers, tests and the benchmark; it
takes device pointers (e.g. ``torch.Tensor.data_ptr()``) and never falls back
to a CPU implementation: if the library is missing it raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libqwmoe.so"

F32, Q8_0, Q4_K, Q6_K, Q8_K, I32 = 0, 8, 12, 14, 15, 26
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292), F32: (1, 4)}

STATUS_TOPK_TIE_SORT, STATUS_BAD_ID, STATUS_BAD_SLOT = 1, 2, 4


class QwmoeError(RuntimeError):
    pass


class Layer(C.Structure):
    """Mirror of ``qwmoe_layer`` (include/qwmoe.h)."""

    _fields_ = [
        ("n_embd", C.c_int64), ("n_expert", C.c_int64), ("n_expert_used", C.c_int64), ("n_ff", C.c_int64),
        ("expert_weights_scale", C.c_float),
        ("router", C.c_void_p),
        ("type_gate", C.c_int), ("type_up", C.c_int), ("type_down", C.c_int),
        ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
        ("gate_nb1", C.c_size_t), ("gate_nb2", C.c_size_t), ("up_nb1", C.c_size_t), ("up_nb2", C.c_size_t),
        ("down_nb1", C.c_size_t), ("down_nb2", C.c_size_t),
        ("n_slots_gate", C.c_int64), ("n_slots_up", C.c_int64), ("n_slots_down", C.c_int64),
        ("slot_gate", C.c_void_p), ("slot_up", C.c_void_p), ("slot_down", C.c_void_p),
        ("resmask", C.c_void_p), ("want_ids", C.c_void_p),
    ]


class SharedExpert(C.Structure):
    """Mirror of ``qwmoe_shared_expert`` (include/qwmoe.h)."""

    _fields_ = [
        ("n_ff", C.c_int64), ("type_gate", C.c_int), ("type_up", C.c_int), ("type_down", C.c_int),
        ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
        ("gate_nb1", C.c_size_t), ("up_nb1", C.c_size_t), ("down_nb1", C.c_size_t),
        ("gate_inp", C.c_void_p),
    ]


class AttnLayer(C.Structure):
    """Mirror of ``qwmoe_attn_layer`` (include/qwmoe.h)."""

    _fields_ = [
        ("n_embd", C.c_int64), ("n_head", C.c_int64), ("n_head_kv", C.c_int64), ("n_embd_head", C.c_int64),
        ("n_rot", C.c_int64), ("rope_freq_base", C.c_float), ("attn_norm", C.c_void_p),
        ("type_q", C.c_int), ("type_k", C.c_int), ("type_v", C.c_int), ("type_o", C.c_int),
        ("wq", C.c_void_p), ("wq_nb1", C.c_size_t), ("wk", C.c_void_p), ("wk_nb1", C.c_size_t),
        ("wv", C.c_void_p), ("wv_nb1", C.c_size_t), ("wo", C.c_void_p), ("wo_nb1", C.c_size_t),
        ("q_norm", C.c_void_p), ("k_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
        ("k_cache", C.c_void_p), ("v_cache", C.c_void_p), ("n_ctx", C.c_int64),
    ]


class GdnLayer(C.Structure):
    """Mirror of ``qwmoe_gdn_layer`` (include/qwmoe.h)."""

    _fields_ = [
        ("n_embd", C.c_int64), ("d_state", C.c_int64), ("n_group", C.c_int64), ("dt_rank", C.c_int64),
        ("d_conv", C.c_int64), ("attn_norm", C.c_void_p),
        ("type_qkv", C.c_int), ("type_gate", C.c_int), ("type_beta", C.c_int), ("type_alpha", C.c_int),
        ("type_out", C.c_int),
        ("w_qkv", C.c_void_p), ("w_qkv_nb1", C.c_size_t), ("w_gate", C.c_void_p), ("w_gate_nb1", C.c_size_t),
        ("w_beta", C.c_void_p), ("w_beta_nb1", C.c_size_t), ("w_alpha", C.c_void_p), ("w_alpha_nb1", C.c_size_t),
        ("w_out", C.c_void_p), ("w_out_nb1", C.c_size_t),
        ("dt_bias", C.c_void_p), ("ssm_a", C.c_void_p), ("conv1d", C.c_void_p), ("ssm_norm", C.c_void_p),
        ("ffn_norm", C.c_void_p), ("conv_state", C.c_void_p), ("ssm_state", C.c_void_p),
    ]


# name -> (restype, argtypes); every exported symbol of include/qwmoe.h
P, I64, SZ, I, F, U64 = C.c_void_p, C.c_int64, C.c_size_t, C.c_int, C.c_float, C.c_uint64
SIGNATURES = {
    "qwmoe_init": (I, [I, SZ]),
    "qwmoe_shutdown": (I, []),
    "qwmoe_strerror": (C.c_char_p, [I]),
    "qwmoe_workspace_high_water": (SZ, []),
    "qwmoe_set_mfma_min_rows": (I, [I]),
    "qwmoe_get_mfma_min_rows": (I, []),
    "qwmoe_set_mfma_form": (I, [I]),
    "qwmoe_get_mfma_form": (I, []),
    "qwmoe_row_size": (SZ, [I, I64]),
    "qwmoe_vec_dot_type": (I, [I]),
    "qwmoe_device_status": (I, [P, P, I]),
    "qwmoe_quantize_act": (I, [P, I, P, I64, I64, I64, SZ, SZ, P]),
    "qwmoe_quantize_chunk": (I, [P, I, P, P, I64, I64]),
    "qwmoe_dequantize": (I, [P, I, P, P, I64]),
    "qwmoe_fill_randn": (I, [P, P, I64, U64, F, F]),
    "qwmoe_mul_mat_id": (I, [P, I, P, I64, I64, I64, SZ, SZ, P, I64, I64, SZ, SZ, P, I64, SZ, P, I64, P, SZ, SZ]),
    "qwmoe_mul_mat_id_noalloc": (I, [P, I, P, I64, I64, I64, SZ, SZ, P, I64, I64, SZ, SZ, P, I64, SZ, P, I64, P, SZ, SZ]),
    "qwmoe_group_by_expert": (I, [P, P, I64, I64, SZ, I64, P, P, P]),
    "qwmoe_router_topk": (I, [P, P, P, I64, I64, I64, I64, SZ, F, F, P, P, P]),
    "qwmoe_router_topk_resident": (I, [P, P, P, I64, I64, I64, I64, SZ, F, F, P, P, P, P, P]),
    "qwmoe_swiglu": (I, [P, P, P, P, I64, I64]),
    "qwmoe_weighted_sum": (I, [P, P, P, P, I64, I64, I64]),
    "qwmoe_rms_norm": (I, [P, P, P, I64, I64, F]),
    "qwmoe_rms_norm_mul": (I, [P, P, P, P, I64, I64, F]),
    "qwmoe_shared_expert_add": (I, [P, P, I64, P, I64, P, P, P]),
    "qwmoe_ffn_layer": (I, [P, P, P, I64, P, F, P, P, P]),
    "qwmoe_attn_seg": (I, [P, P, P, I64, I64, F, P, P]),
    "qwmoe_gdn_seg": (I, [P, P, P, I64, F, P, P]),
    "qwmoe_decoder_layer": (I, [P, P, P, P, I64, I64, F, P, P, P]),
    "qwmoe_decode_stack_create": (I, [P, I, F, P]),
    "qwmoe_decode_stack_run": (I, [P, P, P, P, P, P, P]),
    "qwmoe_decode_stack_status": (I, [P, P, P, I]),
    "qwmoe_decode_stack_free": (None, [P]),
    "qwmoe_decode_stack_kernel": (I, [P]),
    "qwmoe_layer_stack_create": (I, [P, I, F, I, I, P]),
    "qwmoe_layer_stack_run": (I, [P, P, P, I64, P, P, P, P]),
    "qwmoe_layer_stack_free": (None, [P]),
    "qwmoe_layer_stack_captures": (I64, [P]),
    "qwmoe_layer_stack_kernel": (I, [P]),
    "qwmoe_layer_stack_kernel_t1": (I, [P]),
    "qwmoe_layer_stack_status": (I, [P, P, P, I]),
    "qwmoe_slot_table_create": (P, [I, I]),
    "qwmoe_slot_table_free": (None, [P]),
    "qwmoe_slot_table_fill": (I, [P, U64]),
    "qwmoe_slot_table_set": (I, [P, I, I, I, C.c_int32]),
    "qwmoe_slot_table_slot_of": (C.c_int32, [P, I, I, I]),
    "qwmoe_slot_table_row": (P, [P, I, I]),
    "qwmoe_host_argsort_desc": (I, [P, I, P]),
    "qwmoe_gguf_open": (I, [C.c_char_p, P]),
    "qwmoe_gguf_close": (None, [P]),
    "qwmoe_gguf_n_shards": (I, [P]),
    "qwmoe_gguf_shard_info": (I, [P, I, P, P, P]),
    "qwmoe_gguf_n_kv": (I, [P]),
    "qwmoe_gguf_find_key": (I, [P, C.c_char_p]),
    "qwmoe_gguf_kv": (I, [P, I, P, P, P, P, P]),
    "qwmoe_gguf_kv_str": (I, [P, I, U64, P]),
    "qwmoe_gguf_get_u32": (I, [P, C.c_char_p, C.c_uint32, P]),
    "qwmoe_gguf_get_f32": (I, [P, C.c_char_p, F, P]),
    "qwmoe_gguf_get_str": (I, [P, C.c_char_p, C.c_char_p, P]),
    "qwmoe_gguf_n_tensors": (I, [P]),
    "qwmoe_gguf_tensor_at": (I, [P, I, P]),
    "qwmoe_gguf_find_tensor": (I, [P, C.c_char_p, P]),
    "qwmoe_gguf_moe_hparams": (I, [P, P]),
    "qwmoe_gguf_moe_layer_bytes": (I, [P, I, P]),
    "qwmoe_gguf_load_moe_layer": (I, [P, P, I, P, SZ, P]),
    "qwmoe_gguf_shard_path": (I, [P, I, P]),
    "qwmoe_expert_cache_create": (I, [P, I, I, P, P, P]),
    "qwmoe_expert_cache_create_gguf": (I, [P, P, I, P, P]),
    "qwmoe_expert_cache_free": (None, [P]),
    "qwmoe_expert_cache_n_pools": (I, [P]),
    "qwmoe_expert_cache_pool_info": (I, [P, I, P, P, P, P, P, P, P]),
    "qwmoe_expert_cache_pool_of": (I, [P, I, I]),
    "qwmoe_expert_cache_min_slots": (I, [P]),
    "qwmoe_expert_cache_capacity": (I, [P, I]),
    "qwmoe_expert_cache_ensure": (I, [P, I, P, I, P, P, P]),
    "qwmoe_expert_cache_ensure_resident": (I, [P, I, I]),
    "qwmoe_expert_cache_touch": (I, [P, I, I, I]),
    "qwmoe_expert_cache_resident": (I, [P, I, I, I]),
    "qwmoe_expert_cache_verify": (I, [P, P, I, I, I]),
    "qwmoe_expert_cache_resmask": (I, [P, I, P, P]),
    "qwmoe_expert_cache_refill": (I, [P, P, P, I, I, I, P]),
    "qwmoe_plan_slices": (I, [P, I, I, I, I, I, P, P, P, P]),
    "qwmoe_expert_cache_plan_slices": (I, [P, I, P, I, I, P, P]),
    "qwmoe_expert_cache_run_batch": (I, [P, I, P, P, I64, P, F, P, P, P, I, P]),
    "qwmoe_expert_cache_slot_of_row": (P, [P, I, I]),
    "qwmoe_expert_cache_device_row": (P, [P, I, I]),
    "qwmoe_expert_cache_layer": (I, [P, I, P]),
    "qwmoe_expert_cache_get_stats": (I, [P, P]),
    "qwmoe_expert_cache_save_profile": (I, [P, C.c_char_p]),
    "qwmoe_expert_cache_load_prefetch": (I, [P, C.c_char_p, P]),
    "qwmoe_expert_cache_sync": (I, [P]),
    "qwmoe_expert_cache_run_layer": (I, [P, I, P, P, I64, P, F, P, P, P]),
}


class GgufTensorInfo(C.Structure):
    """Mirror of ``qwmoe_gguf_tensor_info``."""

    _fields_ = [("name", C.c_char * 64), ("type", C.c_int32), ("n_dims", C.c_int32), ("ne", C.c_int64 * 4),
                ("offset", C.c_uint64), ("file_offset", C.c_uint64), ("nbytes", C.c_uint64), ("shard", C.c_int32)]


class MoeHparams(C.Structure):
    """Mirror of ``qwmoe_moe_hparams``."""

    _fields_ = [("arch", C.c_char * 32), ("n_layer", C.c_int32), ("n_embd", C.c_int32), ("n_expert", C.c_int32),
                ("n_expert_used", C.c_int32), ("n_ff_exp", C.c_int32), ("expert_weights_scale", C.c_float)]



class ExpertSrc(C.Structure):
    """Mirror of ``qwmoe_expert_src``."""

    _fields_ = [("type", C.c_int32), ("ne0", C.c_int64), ("ne1", C.c_int64), ("host", C.c_void_p),
                ("path", C.c_char_p), ("file_offset", C.c_uint64)]


class ExpertCacheConfig(C.Structure):
    """Mirror of ``qwmoe_expert_cache_config``."""

    _fields_ = [("vram_budget", C.c_size_t), ("n_used", C.c_int32), ("io_threads", C.c_int32), ("flags", C.c_int32)]


class ExpertCacheStats(C.Structure):
    """Mirror of ``qwmoe_expert_cache_stats``."""

    _fields_ = [("hits", C.c_uint64), ("misses", C.c_uint64), ("evictions", C.c_uint64), ("fetch_ms", C.c_double),
                ("fetch_bytes", C.c_uint64)]


CACHE_DRY_RUN, CACHE_COPY_ENGINE = 1, 2
STACK_NO_GRAPH = 1

_lib = None


def lib() -> C.CDLL:
    """Loads libqwmoe.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise QwmoeError(f"{LIB_PATH} is missing: build it with `python -m questwend_amd.build`")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().qwmoe_strerror(rc).decode()
        err = QwmoeError(f"{what}: {msg} ({rc})")
        err.status = rc
        raise err


def row_size(t: int, n: int) -> int:
    qk, bs = BLOCK[t]
    if n % qk:
        raise ValueError(f"row of {n} values is not a multiple of the {qk}-value block")
    return n // qk * bs


def vec_dot_type(t: int) -> int:
    return Q8_0 if t == Q8_0 else Q8_K


from . import ops  # noqa: E402,F401  (torch-facing wrappers)
