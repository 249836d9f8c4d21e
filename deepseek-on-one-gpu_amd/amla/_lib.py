"""ctypes binding of libamla.so (the C ABI declared in include/amla.h).

The library is built in-tree by amla.build; importing this module never builds
and never falls back to anything: a missing library raises immediately.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libamla.so")

c_void_p = ctypes.c_void_p
c_int64 = ctypes.c_int64
c_int = ctypes.c_int
c_size_t = ctypes.c_size_t
c_float = ctypes.c_float


class MlaArgs(ctypes.Structure):
    """Mirror of ``amla_mla_args`` in include/amla.h (same field order)."""
    _fields_ = [
        ("batch", ctypes.c_int32), ("seq_len", ctypes.c_int32), ("hidden", ctypes.c_int32),
        ("heads", ctypes.c_int32), ("q_lora", ctypes.c_int32), ("kv_lora", ctypes.c_int32),
        ("qk_nope", ctypes.c_int32), ("qk_rope", ctypes.c_int32), ("v_dim", ctypes.c_int32),
        ("max_seq", ctypes.c_int32), ("rope_rows", ctypes.c_int32), ("max_context", ctypes.c_int32),
        ("eps", c_float), ("softmax_scale", c_float),
        ("positions", c_void_p), ("hidden_states", c_void_p), ("out", c_void_p),
        ("input_gamma", c_void_p), ("residual", c_void_p),
        ("w_q_a", c_void_p), ("s_q_a", c_void_p), ("w_q_b", c_void_p), ("s_q_b", c_void_p),
        ("w_kv_a", c_void_p), ("s_kv_a", c_void_p), ("w_kv_b", c_void_p), ("s_kv_b", c_void_p),
        ("w_o", c_void_p), ("s_o", c_void_p),
        ("gamma_q", c_void_p), ("gamma_kv", c_void_p),
        ("ckv_cache", c_void_p), ("kpe_cache", c_void_p), ("rope_table", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("attn_out", c_void_p),
    ]


# (name, restype, argtypes) of every exported entry point
SIGNATURES = [
    ("amla_abi_version", c_int, []),
    ("amla_last_error", ctypes.c_char_p, []),
    ("amla_fp8_block_dequant", c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    ("amla_fp8_linear", c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                c_void_p, c_int64, c_void_p, c_size_t, c_void_p]),
    ("amla_fp8_linear_workspace_bytes", c_size_t, [c_int64, c_int64, c_int64]),
    ("amla_fp8_linear_f32", c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                    c_void_p, c_int64, c_void_p, c_size_t, c_void_p]),
    ("amla_rms_norm", c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_float, c_void_p,
                              c_int64, c_void_p]),
    ("amla_apply_rope", c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p]),
    ("amla_mla_decode", c_int, [ctypes.POINTER(MlaArgs), c_void_p]),
    ("amla_mla_prefill", c_int, [ctypes.POINTER(MlaArgs), c_void_p]),
    ("amla_mla_decode_profiled", c_int, [ctypes.POINTER(MlaArgs), c_void_p, ctypes.POINTER(c_void_p)]),
    ("amla_mla_decode_profiled_repeat", c_int, [ctypes.POINTER(MlaArgs), c_void_p, ctypes.POINTER(c_void_p), c_int]),
    ("amla_mla_decode_noalloc", c_int, [ctypes.POINTER(MlaArgs), c_void_p]),
    ("amla_mla_decode_workspace_bytes", c_size_t, [ctypes.POINTER(MlaArgs)]),
    ("amla_mla_prefill_workspace_bytes", c_size_t, [ctypes.POINTER(MlaArgs)]),
    ("amla_silu_mul", c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    ("amla_swiglu", c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                            c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("amla_swiglu_workspace_bytes", c_size_t, [c_int64, c_int64, c_int64]),
    ("amla_moe_route", c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int, c_int, c_int, c_int,
                               c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("amla_moe_route_workspace_bytes", c_size_t, [c_int64, c_int64]),
    ("amla_moe_experts", c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                                 c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("amla_moe_experts_workspace_bytes", c_size_t, [c_int64, c_int64, c_int, c_int64]),
    ("amla_moe_experts_dev", c_int, [c_void_p, c_int64, c_int64, c_int, c_void_p, c_int64, c_int64, c_void_p,
                                     c_void_p, c_void_p, c_size_t, c_void_p]),
    ("amla_moe_experts_dev_workspace_bytes", c_size_t, [c_int64, c_int64, c_int, c_int64, c_int64]),
    ("amla_bf16_logits", c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    ("amla_argmax", c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    ("amla_sample_top_p", c_int, [c_void_p, c_int64, c_int64, c_int64, c_float, c_float, ctypes.c_uint64, c_void_p,
                                  c_void_p]),
    ("amla_sample", c_int, [c_void_p, c_int64, c_int64, c_int64, c_float, c_float, ctypes.c_uint64, c_void_p,
                            c_void_p, c_size_t, c_void_p]),
    ("amla_sample_workspace_bytes", c_size_t, [c_int64, c_int64]),
    ("amla_moe_combine", c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int64, c_float, c_void_p,
                                 c_void_p]),
]

_lib = None


class AmlaError(RuntimeError):
    pass


def lib():
    """Load libamla.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise AmlaError(f"{LIB_PATH} is missing: build it with `python -m amla.build` "
                            "(or __graft_entry__.build()); there is no fallback path")
        h = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _lib = h
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().amla_last_error().decode(errors="replace")
        kind = ValueError if rc < 0 else AmlaError
        raise kind(f"{what} failed ({rc}): {msg}")
