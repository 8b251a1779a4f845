"""ctypes binding of libt2t_attn.so (declarations: include/t2t_attn.h).

The library is the only compute path: if it is missing or cannot be loaded,
every entry point raises.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
import re
from typing import List

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libt2t_attn.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "t2t_attn.h")

T2T_OK = 0
T2T_DTYPE_BF16 = 0
T2T_DTYPE_F32 = 1
T2T_ROWS_STORE, T2T_ROWS_ADD, T2T_ROWS_SWIGLU = 0, 1, 2
ROWS_MAX = 8
TILE = 128
MAX_WORDS = 8
TILE_BITS_WORDS = 1024  # uint32 per tile bitmap slot ([2][128][4])


class T2TTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("stride_b", ctypes.c_int64),
                ("stride_h", ctypes.c_int64), ("stride_t", ctypes.c_int64)]


class T2TBlockMaskC(ctypes.Structure):
    """struct t2t_block_mask (include/t2t_attn.h)."""
    _fields_ = [("mask_batch", ctypes.c_int32), ("num_tiles", ctypes.c_int32)] + [
        (name, ctypes.c_void_p) for name in (
            "kv_num", "kv_idx", "full_kv_num", "full_kv_idx", "q_num", "q_idx",
            "full_q_num", "full_q_idx", "row_order", "col_order", "kv_bits_off",
            "q_bits_slot", "tile_bits")] + [("tile_bits_slots", ctypes.c_int64)]


_lib = None

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SIGS = {
    "t2t_version": ([], ctypes.c_char_p),
    "t2t_last_error": ([], ctypes.c_char_p),
    "t2t_token_inputs": ([_P, _P, _I32, _P, _P, _I32, _P, _I32, _I32, _I32, _P, _P, _P, _P],
                         ctypes.c_int),
    "t2t_mask_meta": ([_P, _P, _P, _I32, _I32, _I32, _P, _P, _P], ctypes.c_int),
    "t2t_attn_fwd": ([_P] * 5 + [_I32] * 6 + [ctypes.c_float, _P, _P], ctypes.c_int),
    "t2t_attn_bwd": ([_P] * 10 + [_I32] * 6 + [ctypes.c_float, _P, _P], ctypes.c_int),
    "t2t_clock_probe": ([_P, _I32, _P, _P], ctypes.c_int),
    "t2t_attn_bwd_noalloc": ([_P] * 9 + [_I32] * 6 + [ctypes.c_float, _P, _P], ctypes.c_int),
    "t2t_attn_bwd_preprocess": ([_P] * 3 + [_I32] * 5 + [_P], ctypes.c_int),
    "t2t_attn_bwd_dkdv": ([_P] * 8 + [_I32] * 6 + [ctypes.c_float, _P, _P], ctypes.c_int),
    "t2t_attn_bwd_dq": ([_P] * 7 + [_I32] * 6 + [ctypes.c_float, _P, _P], ctypes.c_int),
    "t2t_qkv_rope": ([_P, _I64, _I64] + [_I32] * 4 + [_P, _P, _I32, _I32] + [_P] * 4,
                     ctypes.c_int),
    "t2t_qkv_rope_backward": ([_P] * 5 + [_I32] * 6 + [_P, _I64, _I64, _P], ctypes.c_int),
    "t2t_attn_decode_workspace": ([_I32] * 5, ctypes.c_int64),
    "t2t_rms_norm": ([_P, _I64, _P, _I32, _P, _I64, _P, _I32, _I32, ctypes.c_float, _P],
                     ctypes.c_int),
    "t2t_wgrad_workspace": ([_I32, _I32, _I32], ctypes.c_int64),
    "t2t_wgrad": ([_P, _I64, _P, _I64, _P, _I32, _I32, _I32, _I32, _P, _I64, _P], _I32),
    "t2t_swiglu": ([_P, _I64, _P, _I64, _I32, _I32, _P], _I32),
    "t2t_swiglu_backward": ([_P, _I64, _P, _I64, _P, _I64, _I32, _I32, _P], _I32),
    "t2t_ce_rows": ([_P, _P, _I64, _I32, _I64, _P, _I64, _P, _P, _P], _I32),
    "t2t_rms_norm_backward_workspace": ([_I32, _I32], ctypes.c_int64),
    "t2t_rms_norm_backward": ([_P, _I64, _P, _I64, _P, _I32, _P, _P, _I64, _P, _P, _I64, _I32,
                               _I32, _P], ctypes.c_int),
    "t2t_attn_decode": ([_P] * 7 + [_I64] + [_P] * 3 + [_I32] * 9 + [ctypes.c_float, _P, _I64, _P],
                        ctypes.c_int),
    "t2t_rows_linear": ([_P, _I64, _I32, _I32, _P, _I32, _P, _I32, ctypes.c_float, _I32, _P, _I64,
                         _P, _I64, _P, _I32, _P, _I64, _P], ctypes.c_int),
    "t2t_first_input_diff": ([_P] * 8 + [_I64, _I64, _I32, _I32, _P, _P], ctypes.c_int),
    "t2t_rows_qkv_rope": ([_P, _I64, _I32, _I32, _P, _P, _I32, ctypes.c_float, _I32, _I32, _P, _P,
                           _I32, _P, _I32, _P, _P, _P, _I32, _P], ctypes.c_int),
}


def header_functions() -> List[str]:
    """Names of the functions include/t2t_attn.h declares."""
    with open(HEADER_PATH) as f:
        text = f.read()
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(t2t_\w+)\s*\(", text, flags=re.M)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m tagseq2tagseq_amd.build` "
                "(the masked-attention path has no CPU fallback)")
        l = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = res
        _lib = l
    return _lib


def check(rc: int, what: str) -> None:
    if rc != T2T_OK:
        msg = lib().t2t_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def tensor_struct(t) -> T2TTensor:
    """[B, H, T, D] torch tensor with unit stride along D."""
    if t.dim() != 4:
        raise ValueError(f"expected a 4-D [B, H, T, D] tensor, got shape {tuple(t.shape)}")
    if t.stride(3) != 1:
        raise ValueError("the head dimension (last) must have unit stride")
    return T2TTensor(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))
