"""ctypes binding of libmdlarc_hip.so (declared in include/mdlarc_hip.h).

The library must be loaded AFTER torch: both link ``libamdhip64.so.7`` and the dynamic loader then
reuses torch's copy of the HIP runtime, so pointers and streams are shared with torch.  There is no
fallback: if the library is missing every GPU entry point raises.
"""

from __future__ import annotations

import ctypes
import re
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime first)

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libmdlarc_hip.so"
HEADER = _PKG.parent / "include" / "mdlarc_hip.h"

P = c_void_p


class LogitConstraints(ctypes.Structure):
    """``mdl_logit_constraints`` (include/mdlarc_hip.h), field for field."""

    _fields_ = [("disallow_mask", ctypes.c_uint32), ("palette_mask", c_void_p),
                ("palette_penalty", c_float), ("target_shape", c_void_p), ("grid_x", c_void_p),
                ("grid_y", c_void_p), ("shape_penalty", c_float)]


CONS = ctypes.POINTER(LogitConstraints)
# argtypes per entry point, in header order
SIGNATURES: dict[str, tuple[object, list]] = {
    "mdl_version": (c_int, []),
    "mdl_error_string": (ctypes.c_char_p, [c_int]),
    "mdl_embed_rmsnorm": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, P,
                                  c_float, P, P, P, c_int, P]),
    "mdl_decode_embed": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, c_int, P, c_float, P,
                                 P, P, c_int, c_int, P, P, P, P, P, c_int, P]),
    "mdl_add_rmsnorm": (c_int, [P, P, P, c_int, c_int, P, c_float, P, P, c_int, P]),
    "mdl_qkv_rope_cache": (c_int, [P, c_int64, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int,
                                   c_int, c_int, c_int, c_int, c_float, P, P, P, c_int, c_int,
                                   c_int, P, P]),
    "mdl_qkv_rope_cache_packed": (c_int, [P, c_int64, P, P, P, c_int64, P, P, c_int, c_int, c_int,
                                          c_int, c_int, c_int, c_int, c_int, c_int, c_float, P, P,
                                          P, c_int, c_int, P]),
    "mdl_swiglu": (c_int, [P, c_int64, P, P, P, c_int, c_int, P, c_int, P]),
    "mdl_embed_rmsnorm_bf16": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, c_int, P, c_float,
                                       P, P, P]),
    "mdl_qkv_rope_cache_bf16": (c_int, [P, c_int64, P, P, P, c_int, c_int, c_int, c_int, c_int,
                                        c_int, c_int, c_int, c_int, c_int, c_float, P, P, P,
                                        c_int, c_int, P]),
    "mdl_swiglu_bf16": (c_int, [P, c_int64, P, P, P, c_int, c_int, P, P]),
    "mdl_gemm_split": (c_int, [P, c_int64, c_int, P, c_int64, c_int, P, c_int64, c_int, c_int,
                               c_int, c_int, P]),
    "mdl_gemm_split_swiglu": (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, P]),
    "mdl_gemm_norm": (c_int, [P, P, c_float, P, P, P, c_int64, P, c_int, c_int, c_int, c_int,
                              P]),
    "mdl_gemm_norm_qkv": (c_int, [P, P, c_float, P, c_int, c_int, P, P, P, c_int, c_int, c_int,
                                  c_int, c_int, c_int, c_float, P, P, P, c_int, c_int, P, c_int,
                                  P]),
    "mdl_gemm_norm_swiglu": (c_int, [P, P, c_float, P, P, P, P, P, c_int, c_int, c_int, c_int,
                                     P]),
    "mdl_gemm_split_residual": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, P]),
    "mdl_gemm_split_tiles": (c_int, []),
    "mdl_gemm_split_pick": (c_int, [c_int, c_int, c_int]),
    "mdl_prefill_gemm_split": (c_int, [P, c_int64, c_int, c_int, P, P, c_int64, c_int, c_int,
                                       c_int, P]),
    "mdl_prefill_gemm_norm": (c_int, [P, P, c_float, P, P, c_int64, P, c_int, c_int, c_int, P]),
    "mdl_prefill_gemm_norm_swiglu": (c_int, [P, P, c_float, c_int, P, P, P, P, c_int, c_int,
                                             c_int, c_int, P]),
    "mdl_prefill_gemm_split_residual": (c_int, [P, c_int64, c_int, c_int, P, P, P, c_int, c_int,
                                                c_int, P]),
    "mdl_prefill_gemm_norm_qkv": (c_int, [P, P, c_float, P, c_int, c_int, P, P, c_int64, c_int, P,
                                          P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float,
                                          P, P, P, c_int, c_int, c_int, P, P, P]),
    "mdl_tile_matrix": (c_int, [P, c_int64, c_int, c_int, P, P]),
    "mdl_attn_prefill": (c_int, [P, P, P, c_int, c_int, c_int, c_int, c_int, P, P, P, c_int, P,
                                 c_int, P]),
    "mdl_attn_prefill_packed": (c_int, [P, P, P, c_int, c_int, c_int, c_int, c_int, P, P, P, P,
                                        c_int, P, c_int, P]),
    "mdl_attn_prefill_lead": (c_int, [P, c_int64, P, P, P, c_int, c_int, c_int, c_int, c_int,
                                      c_int, c_float, c_int, c_int, c_int, c_int, P, P, P, P,
                                      c_int, P]),
    "mdl_attn_decode_workspace_bytes": (c_int64, [c_int, c_int, c_int, c_int]),
    "mdl_attn_decode": (c_int, [P, P, P, c_int, c_int, c_int, c_int, P, c_int, P, P, P, c_int,
                                P, P, c_int64, c_int, P, c_int, P]),
    "mdl_attn_decode_rope": (c_int, [P, c_int64, P, P, P, c_int, c_int, c_int, c_int, c_int,
                                     c_int, c_float, P, P, c_int, c_int, c_int, c_int, P, c_int,
                                     P, P, P, c_int, P, P, c_int64, c_int, P, c_int, P]),
    "mdl_attn_decode_rope_noalloc": (c_int, [P, c_int64, P, P, P, c_int, c_int, c_int, c_int,
                                             c_int, c_int, c_float, P, P, c_int, c_int, c_int,
                                             c_int, P, c_int, P, P, P, c_int, P, c_int, P, c_int,
                                             P]),
    "mdl_attn_prefill_f32": (c_int, [P, P, P, c_int, c_int, c_int, c_int, c_int, P, P, P, c_int,
                                     P, c_int, P]),
    "mdl_attn_decode_f32": (c_int, [P, P, P, c_int, c_int, c_int, c_int, P, c_int, P, c_int, P, P,
                                    c_int64, c_int, P, c_int, P]),
    "mdl_lm_head": (c_int, [P, P, c_int, c_int, P, c_float, P, c_int, P, P, CONS, c_int, P]),
    "mdl_decode_head": (c_int, [P, c_int, c_int, P, c_float, P, c_int, P, P, P, c_int64, c_int,
                                P, P, c_int, c_int, CONS, c_int, P]),
    "mdl_grid_init": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, P, P, P, P, P, P, P]),
    "mdl_build_prompts": (c_int, [P, c_int64, P, c_int, P, c_int, P, c_int, P, c_int, P, P, P,
                                  P]),
    "mdl_grid_step": (c_int, [P, c_int, c_int, c_int, P, P, P, P, P, P]),
    "mdl_decode_commit": (c_int, [P, c_int, P, c_int64, c_int, P, P, c_int, c_int, P]),
}

_LIB: ctypes.CDLL | None = None


def header_symbols() -> list[str]:
    """Function names declared in include/mdlarc_hip.h."""
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\*?\s+\*?(mdl_[a-z0-9_]+)\(", text, re.M)


def available() -> bool:
    return LIB_PATH.exists()


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m mdlarc_scale_amd.build` "
                "(the HIP kernels are required, there is no fallback path)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(code: int, what: str) -> None:
    if code != 0:
        msg = lib().mdl_error_string(code).decode()
        raise RuntimeError(f"{what} failed: {msg} (code {code})")
