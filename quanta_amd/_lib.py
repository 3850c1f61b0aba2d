"""ctypes binding of the C ABI in include/quanta_moe.h (the in-tree `_qmoe.so`).

The library is loaded on first use. There is no CPU fallback: if the shared object is missing or
cannot be loaded, every entry point raises, naming the build command.
"""

from __future__ import annotations

import ctypes
import re
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("_qmoe.so")
HEADER = Path(__file__).resolve().parent.parent / "include" / "quanta_moe.h"

QMOE_OK, QMOE_EINVAL, QMOE_EHIP = 0, -1, -2
SCORE_SOFTMAX, SCORE_SIGMOID, SCORE_SQRTSOFTPLUS = 0, 1, 2
NORM_NONE, NORM_ALWAYS, NORM_MULTI = 0, 1, 2
FMT_INT4_G64, FMT_BF16, FMT_INT6_G64, FMT_INT3_G64, FMT_INT8_G64 = 0, 1, 2, 3, 4
ROUTER_BF16_TILED, ROUTER_F32 = 0, 1
REGIME_AUTO, REGIME_SMALL, REGIME_LARGE = 0, 1, 2
EPI_SWIGLU, EPI_BF16, EPI_F32 = 0, 1, 2
ACT_SILU, ACT_SILU_CLAMP, ACT_SWIGLU_OAI = 0, 1, 2
SMALL_M_TILE, LARGE_M_TILE = 16, 128
ABI_VERSION = 10
NOALLOC_SCRATCH_BYTES = 64 << 20   # QMOE_NOALLOC_SCRATCH_BYTES


def mtile_upper_bound(mc: int, n_experts: int, m_tile: int) -> int:
    """Most m-tiles a permuted list of mc slots over n_experts can produce."""
    return (mc + m_tile - 1) // m_tile + min(mc, n_experts)


class QmoeConfig(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int32),
        ("n_experts", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("inter", ctypes.c_int32),
        ("shared_inter", ctypes.c_int32),
        ("scoring", ctypes.c_int32),
        ("norm_topk", ctypes.c_int32),
        ("n_group", ctypes.c_int32),
        ("topk_group", ctypes.c_int32),
        ("routed_scale", ctypes.c_float),
        ("expert_format", ctypes.c_int32),
        ("router_format", ctypes.c_int32),
        ("router_rows", ctypes.c_int32),
        ("shared_gated", ctypes.c_int32),
        ("regime", ctypes.c_int32),
        ("act", ctypes.c_int32),
        ("act_alpha", ctypes.c_float),
        ("act_limit", ctypes.c_float),
        ("down_format", ctypes.c_int32),
        ("awq", ctypes.c_int32),
        ("mixed", ctypes.c_int32),
        ("shared_format", ctypes.c_int32),
    ]

    def __init__(self, **kw):
        kw.setdefault("shared_format", FMT_BF16)
        super().__init__(**kw)


class QmoeWeights(ctypes.Structure):
    _fields_ = [
        ("router_w", ctypes.c_void_p),
        ("router_bias", ctypes.c_void_p),
        ("shared_gate_w", ctypes.c_void_p),
        ("gu_codes", ctypes.c_void_p),
        ("gu_sb", ctypes.c_void_p),
        ("dn_codes", ctypes.c_void_p),
        ("dn_sb", ctypes.c_void_p),
        ("sh_gu", ctypes.c_void_p),
        ("sh_dn", ctypes.c_void_p),
        ("sh_gu_sb", ctypes.c_void_p),
        ("sh_dn_sb", ctypes.c_void_p),
        ("awq_gu", ctypes.c_void_p),
        ("awq_dn", ctypes.c_void_p),
        ("gu_rexp", ctypes.c_void_p),
        ("dn_rexp", ctypes.c_void_p),
    ]


DT_BF16, DT_F32 = 0, 1


class QmoeGeneralConfig(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int32),
        ("n_experts", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("inter", ctypes.c_int32),
        ("shared_inter", ctypes.c_int32),
        ("scoring", ctypes.c_int32),
        ("norm_topk", ctypes.c_int32),
        ("n_group", ctypes.c_int32),
        ("topk_group", ctypes.c_int32),
        ("routed_scale", ctypes.c_float),
        ("act", ctypes.c_int32),
        ("act_alpha", ctypes.c_float),
        ("act_limit", ctypes.c_float),
        ("x_dtype", ctypes.c_int32),
        ("gate_dtype", ctypes.c_int32),
        ("experts_packed", ctypes.c_int32),
        ("expert_dtype", ctypes.c_int32),
        ("bits", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("shared_dtype", ctypes.c_int32),
        ("shared_gated", ctypes.c_int32),
        ("shared_gate_dtype", ctypes.c_int32),
        ("dense_all", ctypes.c_int32),
    ]


class QmoeGeneralWeights(ctypes.Structure):
    _fields_ = [
        ("gate", ctypes.c_void_p),
        ("router_bias", ctypes.c_void_p),
        ("gu", ctypes.c_void_p),
        ("gu_scale", ctypes.c_void_p),
        ("gu_bias", ctypes.c_void_p),
        ("dn", ctypes.c_void_p),
        ("dn_scale", ctypes.c_void_p),
        ("dn_bias", ctypes.c_void_p),
        ("sh_gate", ctypes.c_void_p),
        ("sh_up", ctypes.c_void_p),
        ("sh_down", ctypes.c_void_p),
        ("sh_expert_gate", ctypes.c_void_p),
    ]


PROJ_GATE, PROJ_UP, PROJ_DOWN, PROJ_GATE_UP = 0, 1, 2, 3
MAX_STACKS = 12


class QmoeStack(ctypes.Structure):
    _fields_ = [
        ("proj", ctypes.c_int32),
        ("format", ctypes.c_int32),
        ("codes", ctypes.c_void_p),
        ("sb", ctypes.c_void_p),
        ("expert_slot", ctypes.c_void_p),
        ("row_exp", ctypes.c_void_p),
    ]


class QmoeMixed(ctypes.Structure):
    _fields_ = [
        ("n_stacks", ctypes.c_int32),
        ("stacks", QmoeStack * MAX_STACKS),
    ]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> (restype, argtypes); must match include/quanta_moe.h
SIGNATURES = {
    "qmoe_abi_version": (_I, []),
    "qmoe_last_error": (ctypes.c_char_p, []),
    "qmoe_forward_workspace": (ctypes.c_size_t, [ctypes.POINTER(QmoeConfig), _I64]),
    "qmoe_forward": (_I, [ctypes.POINTER(QmoeConfig), ctypes.POINTER(QmoeWeights), _P, _I64, _P, _P,
                          ctypes.c_size_t, _P]),
    "qmoe_forward_noalloc": (_I, [ctypes.POINTER(QmoeConfig), ctypes.POINTER(QmoeWeights), _P, _I64,
                                  _P, _P]),
    "qmoe_forward_mixed": (_I, [ctypes.POINTER(QmoeConfig), ctypes.POINTER(QmoeWeights),
                                ctypes.POINTER(QmoeMixed), _P, _I64, _P, _P, ctypes.c_size_t, _P]),
    "qmoe_forward_residual_workspace": (ctypes.c_size_t, [ctypes.POINTER(QmoeConfig), _I64]),
    "qmoe_forward_residual": (_I, [ctypes.POINTER(QmoeConfig), ctypes.POINTER(QmoeWeights), _P, _P, _F,
                                   _I64, _P, _P, ctypes.c_size_t, _P]),
    "qmoe_rmsnorm": (_I, [_P, _P, _I64, _I, _F, _P, _P]),
    "qmoe_router_topk": (_I, [_P, _I64, _P, _I64, _I, _I, _I, _I, _I, _I, _F, _I, _P, _P, _P, _P]),
    "qmoe_router_logits_f32": (_I, [_P, _P, _P, _I64, _I, _I, _P, _I64, _P]),
    "qmoe_router_workspace": (ctypes.c_size_t, [_I64, _I]),
    "qmoe_router": (_I, [_P, _P, _I, _P, _P, _I64, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P,
                         ctypes.c_size_t, _P]),
    "qmoe_permute": (_I, [_P, _I64, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "qmoe_grouped_qmm": (_I, [_P, _I64, _P, _I, _I64, _P, _P, _P, _I, _I64, _I, _I, _I, _P, _P, _P,
                              _I, _I, _F, _F, _P, _I, _I, _P, ctypes.c_size_t, _P]),
    "qmoe_grouped_qmm_workspace": (ctypes.c_size_t, [_I64, _I, _I, _I]),
    "qmoe_combine": (_I, [_P, _P, _P, _I64, _I, _I, _P, _P, _P, _P]),
    "qmoe_dequant": (_I, [_P, _P, _P, _I64, _I64, _I, _I, _P, _P]),
    "qmoe_tile_int4": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P, _P, _P]),
    "qmoe_row_exponents": (_I, [_P, _P, _I64, _I64, _I64, _I, _I, _P, _P]),
    "qmoe_dequant_tiled": (_I, [_P, _P, _I64, _I64, _I64, _P, _P]),
    "qmoe_tile_int6": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P, _P, _P]),
    "qmoe_tile_int8": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P, _P, _P]),
    "qmoe_tile_int3": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P, _P, _P]),
    "qmoe_tile_bf16": (_I, [_P, _I64, _I64, _I64, _P, _P]),
    "qmoe_forward_general_workspace": (ctypes.c_size_t, [ctypes.POINTER(QmoeGeneralConfig), _I64]),
    "qmoe_forward_general": (_I, [ctypes.POINTER(QmoeGeneralConfig), ctypes.POINTER(QmoeGeneralWeights),
                                  _P, _I64, _P, _P, ctypes.c_size_t, _P]),
    "qmoe_set_decode_flow": (_I, [_I]),
    "qmoe_set_route_tail": (_I, [_I]),
    "qmoe_flow_timeouts": (ctypes.c_uint32, []),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def header_symbols() -> list[str]:
    """Function names declared in include/quanta_moe.h."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qmoe_[a-z0-9_]+)\s*\(", text)))


def load() -> ctypes.CDLL:
    """Load `_qmoe.so` (once) and attach the ctypes signatures. Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"quanta_amd HIP extension not built ({LIB_PATH} missing); run "
                "`python -m quanta_amd.build` (or __graft_entry__.build()) first")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.qmoe_abi_version() != ABI_VERSION:
            raise RuntimeError("quanta_amd: ABI version mismatch; rebuild the extension")
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Translate a C-ABI status into a Python exception (ValueError for bad arguments)."""
    if rc == QMOE_OK:
        return
    msg = load().qmoe_last_error().decode(errors="replace")
    if rc == QMOE_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error: {msg}")
