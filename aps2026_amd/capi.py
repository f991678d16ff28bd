"""ctypes binding of the C ABI declared in include/aps_moe.h.

The shared library is built in-tree (``aps2026_amd/libaps_moe.so``, see
aps2026_amd/build.py).  Loading fails loudly if it is missing: there is no
fallback implementation of any entry point.
"""
from __future__ import annotations

import ctypes
import os
import re
from typing import List

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libaps_moe.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "aps_moe.h")

APS_OK = 0
APS_ERR_SHAPE = -1
APS_ERR_HANDLE = -2
APS_ERR_DTYPE = -3
APS_ERR_HIP = -4
APS_ERR_ARG = -5
APS_ERR_WORKSPACE = -6

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_E4M3 = 2

_c_vp = ctypes.c_void_p
_c_vpp = ctypes.POINTER(ctypes.c_void_p)
_c_fpp = ctypes.POINTER(ctypes.c_void_p)


class WeightsDesc(ctypes.Structure):
    _fields_ = [
        ("num_experts", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("ffn", ctypes.c_int32),
        ("src_dtype", ctypes.c_int32),
        ("compute_dtype", ctypes.c_int32),
        ("w1", _c_vpp),
        ("w3", _c_vpp),
        ("w2", _c_vpp),
        ("w1_scale", _c_fpp),
        ("w3_scale", _c_fpp),
        ("w2_scale", _c_fpp),
    ]


class WsLayout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in (
        "total_bytes", "logits", "routes", "tile_counts", "counts", "offsets",
        "assignment_rows", "route_positions", "act", "act_scale", "y", "xq", "xq_scale", "actq",
        "tile_counts0", "slot1", "slot_rows", "slot_tokens")]


class ApsError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


_lib = None


def declared_symbols() -> List[str]:
    """Function names declared in include/aps_moe.h."""
    text = open(HEADER_PATH).read()
    return sorted(set(re.findall(r"^APS_API\s+[\w\s\*]+?\b(aps_\w+)\s*\(", text, flags=re.M)))


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    L = ctypes.CDLL(LIB_PATH)
    i32, i64, u64, sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t
    L.aps_moe_last_error.restype = ctypes.c_char_p
    L.aps_moe_abi_version.restype = ctypes.c_int
    L.aps_moe_weights_register.argtypes = [ctypes.POINTER(WeightsDesc), _c_vp, ctypes.POINTER(u64)]
    L.aps_moe_weights_release.argtypes = [u64]
    L.aps_moe_workspace_layout.argtypes = [u64, i64, ctypes.POINTER(WsLayout)]
    L.aps_moe_dispatch_workspace_size.argtypes = [i64, i32]
    L.aps_moe_dispatch_workspace_size.restype = sz
    L.aps_router_logits.argtypes = [_c_vp, i32, _c_vp, i64, i32, i32, _c_vp, _c_vp]
    L.aps_moe_route_top2.argtypes = [_c_vp, i64, i32, _c_vp, _c_vp]
    L.aps_moe_dispatch.argtypes = [_c_vp, i64, i32, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, sz, _c_vp]
    L.aps_moe_expert_ffn.argtypes = [u64, _c_vp, i32, i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]
    L.aps_moe_ffn_up.argtypes = [u64, _c_vp, i32, i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]
    L.aps_moe_ffn_down.argtypes = [u64, _c_vp, _c_vp, i64, _c_vp, _c_vp, _c_vp]
    L.aps_moe_combine.argtypes = [_c_vp, i32, _c_vp, i64, i32, _c_vp, i32, _c_vp]
    L.aps_moe_forward_grouped.argtypes = [u64, _c_vp, i32, _c_vp, i64, _c_vp, i32, _c_vp, sz, _c_vp]
    L.aps_moe_forward.argtypes = [u64, _c_vp, i32, _c_vp, i64, _c_vp, i32, _c_vp, sz, _c_vp]
    L.aps_mlp_workspace_size.argtypes = [u64, i64]
    L.aps_mlp_workspace_size.restype = sz
    L.aps_mlp_forward.argtypes = [u64, _c_vp, i32, i64, _c_vp, _c_vp, sz, _c_vp]
    L.aps_quantise_rows_e4m3.argtypes = [_c_vp, i64, i32, _c_vp, i64, _c_vp, i64, _c_vp]
    L.aps_moe_ffn_up_fp8.argtypes = [u64, _c_vp, _c_vp, i64, _c_vp, _c_vp, _c_vp, _c_vp]
    L.aps_moe_ffn_down_fp8.argtypes = [u64, _c_vp, _c_vp, i64, _c_vp, _c_vp, _c_vp]
    L.aps_layer_norm.argtypes = [_c_vp, _c_vp, _c_vp, i64, i32, ctypes.c_float, _c_vp, _c_vp]
    L.aps_add_layer_norm.argtypes = [_c_vp, _c_vp, _c_vp, _c_vp, i64, i32, ctypes.c_float, _c_vp, _c_vp]
    L.aps_gather_rows.argtypes = [_c_vp, i64, i64, _c_vp, i64, _c_vp, _c_vp]
    L.aps_prefix_ancestors.argtypes = [_c_vp, _c_vp, _c_vp, i64, i64, _c_vp, _c_vp]
    L.aps_linear.argtypes = [_c_vp, _c_vp, _c_vp, i64, i32, i32, _c_vp, _c_vp]
    L.aps_linear_multi.argtypes = [_c_vp, i64, i32, i32, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]
    L.aps_linear_tc_packed_bytes.argtypes = [i32, i32]
    L.aps_linear_tc_packed_bytes.restype = sz
    L.aps_linear_tc_prepare.argtypes = [_c_vp, i32, i32, _c_vp, sz, _c_vp]
    L.aps_linear_tc_split.argtypes = [_c_vp, i64, i32, _c_vp, _c_vp]
    L.aps_linear_tc.argtypes = [_c_vp, i64, i32, _c_vp, _c_vp, i32, i32, _c_vp, _c_vp]
    L.aps_linear_tc_multi.argtypes = [_c_vp, i64, i32, i32, _c_vp, _c_vp, _c_vp, i32, _c_vp, _c_vp]
    L.aps_rope_table.argtypes = [i64, i32, ctypes.c_float, _c_vp, _c_vp]
    L.aps_rope_tree.argtypes = [_c_vp, _c_vp, _c_vp, i64, i32, i32, i32, _c_vp, _c_vp, i64, _c_vp]
    L.aps_attention_tree.argtypes = [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, i64, i64, i32, i32, i32, i32, _c_vp]
    L.aps_attention_packed.argtypes = [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, i64, i64, i32, i32, i32, i32,
                                       _c_vp]
    L.aps_add_inplace.argtypes = [_c_vp, _c_vp, i64, _c_vp]
    L.aps_add_bias_inplace.argtypes = [_c_vp, _c_vp, i64, i32, _c_vp]
    L.aps_silu_mul.argtypes = [_c_vp, _c_vp, _c_vp, i64, _c_vp]
    L.aps_zero.argtypes = [_c_vp, i64, _c_vp]
    L.aps_moe_forward_noalloc.argtypes = [u64, _c_vp, i32, _c_vp, i64, _c_vp, i32, _c_vp]
    L.aps_moe_noalloc_scratch_bytes.argtypes = []
    L.aps_moe_noalloc_scratch_bytes.restype = sz
    L.aps_prefix_dedup.argtypes = [_c_vp, _c_vp, i64, i64, i64, _c_vp, _c_vp, _c_vp, _c_vp, i64,
                                   ctypes.POINTER(i64)]
    for name in ("aps_moe_weights_register", "aps_moe_weights_release", "aps_moe_workspace_layout",
                 "aps_router_logits", "aps_moe_route_top2", "aps_moe_dispatch", "aps_moe_expert_ffn",
                 "aps_moe_combine", "aps_moe_forward_grouped", "aps_moe_forward", "aps_moe_ffn_up",
                 "aps_moe_ffn_down", "aps_mlp_forward", "aps_quantise_rows_e4m3", "aps_moe_ffn_up_fp8",
                 "aps_moe_ffn_down_fp8", "aps_layer_norm", "aps_add_layer_norm", "aps_gather_rows",
                 "aps_prefix_dedup", "aps_prefix_ancestors", "aps_linear", "aps_linear_multi", "aps_linear_tc_prepare", "aps_linear_tc_split", "aps_linear_tc", "aps_linear_tc_multi",
                 "aps_rope_table", "aps_rope_tree", "aps_attention_tree",
                 "aps_attention_packed", "aps_add_inplace", "aps_add_bias_inplace", "aps_silu_mul", "aps_zero",
                 "aps_moe_forward_noalloc"):
        getattr(L, name).restype = ctypes.c_int
    _lib = L
    return L


def last_error() -> str:
    return lib().aps_moe_last_error().decode()


def check(rc: int) -> None:
    if rc != APS_OK:
        raise ApsError(rc, last_error())
