"""ctypes binding to libaneforge_hip.so (the C ABI declared in include/aneforge_hip.h).

The reference binds its native dispatch library the same way (ctypes over a C ABI,
aneforge/_runtime.py:20-92); here the library holds hand-written HIP kernels for gfx950.
Every entry point returns 0 on success or a negative code; `call` turns a failure into a
RuntimeError carrying afx_last_error(), mirroring the reference's rc -> RuntimeError
convention (aneforge/_runtime.py:160-175).

There is deliberately no CPU fallback: if the library or a GPU is missing, the first call
raises."""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
_LIB_NAME = "libaneforge_hip.so"

_vp, _i, _ll, _f, _ip, _fp = C.c_void_p, C.c_int, C.c_longlong, C.c_float, C.POINTER(C.c_int), C.POINTER(C.c_float)
_llp = C.POINTER(C.c_longlong)

# name -> (restype, argtypes).  Kept in the same order as include/aneforge_hip.h.
SIGNATURES: dict[str, tuple] = {
    "afx_last_error": (C.c_char_p, []),
    "afx_abi_version": (_i, []),
    "afx_device_info": (_i, [_i, _ip, _ip, _ip, _ip]),
    "afx_stream_sync": (_i, [_vp]),
    "afx_graph_begin": (_i, [_vp]),
    "afx_graph_end": (_i, [_vp, C.POINTER(_vp)]),
    "afx_graph_launch": (_i, [_vp, _vp]),
    "afx_graph_destroy": (_i, [_vp]),
    "afx_event_create": (_i, [C.POINTER(_vp)]),
    "afx_event_record": (_i, [_vp, _vp]),
    "afx_event_elapsed_ms": (_i, [_vp, _vp, _fp]),
    "afx_event_destroy": (_i, [_vp]),
    # weight-streaming linear layers
    "afx_linear": (_i, [_i, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp, _ll, _vp]),
    "afx_linear_rms": (_i, [_i, _vp, _vp, _vp, _i, _vp, _f, _vp, _i, _i, _i, _i, _vp, _i, _i, _vp]),
    "afx_lm_head": (_i, [_i, _vp, _vp, _vp, _vp, _f, _vp, _i, _i, _vp, _vp, _vp]),
    "afx_linear_swiglu": (_i, [_i, _vp, _vp, _vp, _i, _vp, _f, _i, _vp, _i, _i, _i, _i, _i, _vp]),
    "afx_linear_geglu": (_i, [_i, _vp, _vp, _vp, _i, _vp, _f, _i, _vp, _i, _i, _i, _i, _i, _vp]),
    "afx_qkv_rope_kv": (_i, [_i, _vp, _vp, _vp, _i, _vp, _f, _i, _vp, _i, _i, _i, _i, _vp, _vp, _i, _vp,
                             _vp, _i, _vp, _vp, _ll, _ll, _i, _i, _i, _i, _vp]),
    # codecs
    "afx_q4_0_repack": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "afx_q4_k_repack": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "afx_q6_k_repack": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "afx_q4_0_unpack": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "afx_dequant": (_i, [_i, _vp, _vp, _vp, _i, _i, _vp]),
    "afx_dequant_f16": (_i, [_i, _vp, _vp, _vp, _ll, _i, _i, _vp]),
    # attention
    "afx_decode_attn_ws_bytes": (_ll, [_i, _i, _i, _i, _i, _i]),
    "afx_sample": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _ll, _vp]),
    "afx_sample_ws_bytes": (_ll, [_i]),
    "afx_decode_attn": (_i, [_vp, _vp, _vp, _vp, _ll, _ll, _ll, _ll, _i, _i, _i, _i, _i, _vp, _i, _vp, _ll,
                             _i, _f, _vp, _ll, _i, _vp]),
    "afx_decode_attn_noalloc": (_i, [_vp, _vp, _vp, _vp, _ll, _ll, _ll, _ll, _i, _i, _i, _i, _i, _vp, _i, _vp,
                                     _ll, _i, _f, _i, _vp]),
    # norms, rope, sampling, generic tensor ops
    "afx_rmsnorm": (_i, [_vp, _i, _vp, _f, _vp, _i, _i, _i, _vp]),
    "afx_rope": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _i, _i, _vp]),
    "afx_head_norm_rope": (_i, [_vp, _ll, _ll, _i, _vp, _i, _i, _i, _i, _vp, _f, _vp, _vp, _i, _vp]),
    "afx_embed": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "afx_decode_advance": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp,
                                _i, _i, _vp]),
    "afx_argmax": (_i, [_vp, _i, _i, _vp, _vp]),
    "afx_fill_i32": (_i, [_vp, _i, _i, _vp]),
    "afx_fill_f16": (_i, [_vp, _ll, _f, _vp]),
    "afx_ew_binary": (_i, [_i, _vp, _llp, _vp, _llp, _vp, _i, _ip, _vp]),
    "afx_ew_select": (_i, [_vp, _llp, _vp, _llp, _vp, _llp, _vp, _i, _ip, _vp]),
    "afx_ew_unary": (_i, [_i, _vp, _vp, _ll, _f, _f, _vp]),
    "afx_copy_strided": (_i, [_vp, _llp, _vp, _llp, _i, _ip, _vp]),
    "afx_softmax": (_i, [_vp, _vp, _i, _i, _vp]),
    "afx_reduce": (_i, [_i, _vp, _vp, _i, _i, _vp]),
    "afx_bmm_f16": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _ll, _ll, _ll, _vp]),
    # mixture of experts
    "afx_moe_topk": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    "afx_moe_gateup": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _i, _vp]),
    "afx_moe_down": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _ll, _vp]),
    "afx_topk_mask": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    # batched prefill
    "afx_gemm": (_i, [_i, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _vp, _i, _vp]),
    "afx_qkv_split_rope": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp, _i, _vp, _vp, _ll, _i, _vp]),
    "afx_prefill_attn": (_i, [_vp, _i, _vp, _vp, _ll, _i, _vp, _i, _i, _i, _i, _i, _i, _f, _vp]),
    "afx_moe_combine": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "afx_moe_route": (_i, [_vp, _i, _vp, _f, _vp, _i, _i, _i, _i, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "afx_moe_route_sync_words": (_i, []),
    "afx_moe_down_combine": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _ll, _vp, _vp, _vp,
                                  _vp, _vp]),
}

_lib = None


def lib_path() -> Path:
    env = os.environ.get("AFX_LIB")
    return Path(env) if env else _PKG / _LIB_NAME


def load() -> C.CDLL:
    """Load and bind the library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    p = lib_path()
    if not p.is_file():
        raise RuntimeError(f"{p} not found: build it first (python -m aneforge_amd._build)")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().afx_last_error()
    return msg.decode(errors="replace") if msg else ""


def call(name: str, *args) -> int:
    """Invoke an int-returning entry point; raise RuntimeError on a negative return code."""
    rc = getattr(load(), name)(*args)
    if rc < 0:
        raise RuntimeError(f"{name} failed (rc={rc}): {last_error()}")
    return rc


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
