"""ctypes binding of ``libfgs_moe.so`` (C ABI declared in include/fgs_moe.h).

The library is built in-tree (``make -C flaggems-sglang_amd/csrc``) and
lives next to this file. There is no fallback: if the library is missing or
fails to load, every op raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

FGS_OK = 0
FGS_EINVAL = -1
FGS_EUNSUPPORTED = -2
FGS_ELAUNCH = -3

QMODE_BF16 = 0
QMODE_FP8_BLOCK = 1
QMODE_INT8_CHANNEL = 2

SCORING_SOFTMAX = 0
SCORING_SIGMOID = 1

FLAG_ROUTER_WEIGHT_ON_INPUT = 0x1
FLAG_ACT_GELU = 0x2
FLAG_SEPARATE_QUANT = 0x8
FLAG_FORCE_DECODE = 0x100
FLAG_FORCE_PREFILL = 0x200
FLAG_SEPARATE_SUM = 0x400
FLAG_FOLD_SUM = 0x800
TILED_CONFIGS = 5  # row blocks 256, 128, 64, 32, 160
ROUTING_BLOCK_MS = (16, 32, 64, 128)  # tile tables of fgs_moe_topk_to_routing
NOALLOC_SCRATCH_BYTES = 64 << 20  # FGS_NOALLOC_SCRATCH_BYTES


def flag_tile(cfg: int) -> int:
    """Schedule flag forcing tiled configuration ``cfg`` (FGS_FLAG_TILE)."""
    return ((cfg + 1) & 0x7) << 12

LIB_NAME = "libfgs_moe.so"

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64

# name -> (restype, argtypes); mirrors include/fgs_moe.h one to one.
SIGNATURES = {
    "fgs_moe_version": (ctypes.c_char_p, []),
    "fgs_moe_last_error": (ctypes.c_char_p, []),
    "fgs_moe_align_max_padded": (_i64, [_i64, _i32, _i32]),
    "fgs_moe_align_block_size": (
        _i32,
        [_c_void_p, _i64, _i32, _i32, _c_void_p, _c_void_p, _c_void_p, _i64,
         _c_void_p, _i64, _c_void_p],
    ),
    "fgs_moe_align_scratch_bytes": (_i64, [_i64, _i32]),
    "fgs_moe_routing_max_tiles": (_i64, [_i64, _i32]),
    "fgs_moe_routing_workspace_bytes": (_i64, [_i64, _i32]),
    "fgs_moe_topk_to_routing": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _i32, _i32, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _i64,
         _c_void_p],
    ),
    "fgs_moe_routing_to_topk": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i32, _c_void_p, _c_void_p,
         _c_void_p],
    ),
    "fgs_moe_silu_and_mul": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p]),
    "fgs_moe_sum": (_i32, [_c_void_p, _c_void_p, _i64, _i32, _i64, _c_void_p]),
    "fgs_moe_topk_gating": (
        _i32, [_c_void_p, _i32, _i64, _i32, _i32, _i32, _i32, _c_void_p, _c_void_p,
               _c_void_p]
    ),
    "fgs_moe_quant_fp8_group": (
        _i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p]
    ),
    "fgs_moe_quant_int8_token": (
        _i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p]
    ),
    "fgs_moe_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32, _i32, _i32, _i32]),
    "fgs_moe_validate": (_i32, [_i64, _i64, _i64, _i32, _i32, _i32, _i32, _i64]),
    "fgs_moe_schedule": (_i32, [_i64, _i64, _i64, _i32, _i32, _i32, _i32, _c_void_p, _i32]),
    "fgs_moe_fused_bf16": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64,
         _i64, _i32, _i32, _i32, _c_void_p, _i64, _c_void_p, _c_void_p],
    ),
    "fgs_moe_fused_bf16_noalloc": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64,
         _i64, _i32, _i32, _i32, _c_void_p, _c_void_p],
    ),
    "fgs_moe_fused_bf16_bias": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _i64, _i64, _i64, _i32, _i32, _i32, ctypes.c_float,
         ctypes.c_float, _c_void_p, _i64, _c_void_p, _c_void_p],
    ),
    "fgs_moe_fused_quant_bias": (
        _i32,
        [_i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i32, _i32, _i32,
         ctypes.c_float, ctypes.c_float, _c_void_p, _i64, _c_void_p, _c_void_p],
    ),
    "fgs_moe_fused_routed": (
        _i32,
        [_i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, ctypes.c_float, ctypes.c_float, _c_void_p, _c_void_p, _c_void_p,
         _i64, _i64, _i64, _i32, _i32, _i32, _c_void_p, _i64, _c_void_p, _c_void_p],
    ),
    "fgs_moe_fused_fp8_block": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i32,
         _c_void_p, _c_void_p, _i64, _i64, _i64, _i32, _i32, _i32, _c_void_p,
         _i64, _c_void_p, _c_void_p],
    ),
    "fgs_moe_fused_int8_channel": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _i64, _i64, _i64, _i32, _i32, _i32, _c_void_p, _i64,
         _c_void_p, _c_void_p],
    ),
    "fgs_moe_profile_enable": (_i32, [_i32]),
    "fgs_moe_profile_read": (_i32, [_c_void_p, _i32]),
}

PROFILE_STAGES = ("align", "quant_x", "gemm1", "quant_a2", "gemm2", "moe_sum")

_lib = None
_lock = threading.Lock()


def lib_path() -> str:
    """Path of the shared library (``FGS_MOE_LIB`` overrides)."""
    env = os.environ.get("FGS_MOE_LIB")
    if env:
        return env
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not os.path.exists(path):
                raise RuntimeError(
                    f"{LIB_NAME} not found at {path}; build it with "
                    "`make -C flaggems-sglang_amd/csrc` (or "
                    "__graft_entry__.build())"
                )
            lib = ctypes.CDLL(path)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def last_error() -> str:
    return load().fgs_moe_last_error().decode()


def check(rc: int, what: str) -> None:
    """Map a C status code onto the Python exception the op raises."""
    if rc == FGS_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == FGS_EINVAL:
        raise ValueError(msg)
    if rc == FGS_EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def schedule(m: int, hidden: int, inter: int, num_experts: int, topk: int,
             qmode: int = QMODE_BF16, flags: int = 0) -> str:
    """The schedule a fused call of this problem runs (``fgs_moe_schedule``):
    "direct", "direct_sum", "stream mt=T" or "tiled ..."."""
    buf = ctypes.create_string_buffer(96)
    check(load().fgs_moe_schedule(m, hidden, inter, num_experts, topk, qmode, flags,
                                  buf, len(buf)), "schedule")
    return buf.value.decode()
