"""ctypes binding of libgodwit_hip.so (the C ABI in include/godwit_hip.h).

Loading fails loudly: there is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# GODWIT_TRACE_LIB=1 loads the phase-stamped build (build.py --trace) instead.
LIB_PATH = os.path.join(HERE, "libgodwit_hip_trace.so" if os.environ.get("GODWIT_TRACE_LIB") == "1"
                        else "libgodwit_hip.so")

(GW_OK, GW_ERR_ARG, GW_ERR_SHAPE, GW_ERR_OOM, GW_ERR_HIP, GW_ERR_NO_DEVICE, GW_ERR_UNSUPPORTED,
 GW_ERR_EXCHANGE) = range(8)
STATUS_NAMES = {0: "GW_OK", 1: "GW_ERR_ARG", 2: "GW_ERR_SHAPE", 3: "GW_ERR_OOM", 4: "GW_ERR_HIP",
                5: "GW_ERR_NO_DEVICE", 6: "GW_ERR_UNSUPPORTED", 7: "GW_ERR_EXCHANGE"}
F32, F16, BF16 = 0, 1, 2
ACT_GPTOSS_CLAMPED_GLU, ACT_SILU = 0, 1
SECTION_COUNT = 6
STATIC_SCRATCH_BYTES = 8 << 20   # GW_STATIC_SCRATCH_BYTES

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t


class ExpertLayoutC(ctypes.Structure):
    _fields_ = [("hidden_size", _I64), ("intermediate_size", _I64), ("expert_count", _I64),
                ("offsets", _I64 * SECTION_COUNT), ("sizes", _I64 * SECTION_COUNT),
                ("stride", _I64), ("page_size", _I64)]


class ExpertWeightsC(ctypes.Structure):
    _fields_ = [("buffer", _P), ("offsets", _I64 * SECTION_COUNT)]


class AssignmentC(ctypes.Structure):
    _fields_ = [("weights", ExpertWeightsC), ("token", _I32), ("routing_weight", _F)]


class PrefillViewC(ctypes.Structure):
    _fields_ = [("routing_ids", _P), ("routing_weights", _P), ("activations", _P),
                ("activation_plane", ctypes.c_int64), ("expert_outputs", _P),
                ("tokens", ctypes.c_int32), ("top_k", ctypes.c_int32)]


class MoeLayerArgsC(ctypes.Structure):
    _fields_ = [("experts_base", _P), ("expert_stride", _I64), ("expert_count", _I64),
                ("top_k", _I64), ("logits", _P), ("router_weight", _P),
                ("router_weight_dtype", _I), ("router_bias", _P), ("router_bias_dtype", _I),
                ("x", _P), ("x_dtype", _I), ("tokens", _I32), ("out", _P), ("out_bf16", _P),
                ("routing_ids", _P), ("routing_weights", _P)]


class ModelInfoC(ctypes.Structure):
    _fields_ = [("format_version", _I64), ("layer_count", _I64), ("expert_count", _I64),
                ("expert_stride", _I64), ("section_offset", _I64 * 6),
                ("section_length", _I64 * 6), ("hidden_size", _I64),
                ("intermediate_size", _I64), ("experts_per_token", _I64),
                ("rms_norm_epsilon", ctypes.c_float), ("activation_limit", ctypes.c_float),
                ("activation_alpha", ctypes.c_float), ("activation", _I),
                ("expert_bias", _I32), ("router_bias", _I32)]


class MoeBlockArgsC(ctypes.Structure):
    _fields_ = [("layer", MoeLayerArgsC), ("stream", _P), ("norm_weight", _P),
                ("norm_weight_dtype", _I), ("epsilon", ctypes.c_float)]


# name -> (restype, argtypes).  This table is also the list of exported
# symbols the CPU tests check against include/godwit_hip.h.
SIGNATURES = {
    "gw_last_error": (ctypes.c_char_p, []),
    "gw_version": (ctypes.c_char_p, []),
    "gw_device_count": (_I, [ctypes.POINTER(_I)]),
    "gw_context_create": (_I, [_I, ctypes.POINTER(_P)]),
    "gw_context_destroy": (_I, [_P]),
    "gw_context_synchronize": (_I, [_P]),
    "gw_context_stream": (_P, [_P]),
    "gw_context_cu_count": (_I, [_P, ctypes.POINTER(_I)]),
    "gw_context_set_profiling": (_I, [_P, _I]),
    "gw_context_profile_read": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                     ctypes.POINTER(_I64)]),
    "gw_context_profile_reset": (_I, [_P]),
    "gw_malloc": (_I, [_P, _SZ, ctypes.POINTER(_P)]),
    "gw_free": (_I, [_P, _P]),
    "gw_memcpy_htod": (_I, [_P, _P, _P, _SZ]),
    "gw_memcpy_dtoh": (_I, [_P, _P, _P, _SZ]),
    "gw_memcpy_dtod": (_I, [_P, _P, _P, _SZ]),
    "gw_memset_zero": (_I, [_P, _P, _SZ]),
    "gw_memcpy_dtod_async": (_I, [_P, _P, _P, _SZ]),
    "gw_fill_uniform_u8": (_I, [_P, _P, _SZ, _SZ, _SZ, _I, _I, ctypes.c_uint64]),
    "gw_fill_normal": (_I, [_P, _P, _I, _SZ, _SZ, _SZ, _F, _F, ctypes.c_uint64]),
    "gw_expert_layout_init": (_I, [_I64, _I64, _I64, ctypes.POINTER(ExpertLayoutC)]),
    "gw_mxfp4_dequant": (_I, [_P, _P, _P, _I64, _P]),
    "gw_mxfp4_gemv": (_I, [_P, _P, _P, _P, _I, _P, _I64, _I64]),
    "gw_mxfp4_gemv_bias": (_I, [_P, _P, _P, _P, _I, _P, _I, _P, _I64, _I64]),
    "gw_expert_activation": (_I, [_P, _I, _P, _P, _I64, _F, _F]),
    "gw_expert_accumulate": (_I, [_P, _P, _P, _F, _I64]),
    "gw_router_logits": (_I, [_P, _P, _I, _P, _I, _P, _I, _P, _I64, _I64, _I32]),
    "gw_router_select": (_I, [_P, _I64, _I64, _P, _P]),
    "gw_expert_runner_create": (_I, [_P, _I64, _I64, _I, _F, _F, ctypes.POINTER(_P)]),
    "gw_expert_runner_destroy": (_I, [_P]),
    "gw_expert_runner_set_bias_dtype": (_I, [_P, _I]),
    "gw_expert_runner_section_offsets": (_I, [_P, _I64 * SECTION_COUNT]),
    "gw_expert_runner_sync_errors": (_I, [_P, ctypes.POINTER(ctypes.c_uint32)]),
    "gw_expert_runner_set_wait_limit": (_I, [_P, ctypes.c_uint32]),
    "gw_expert_runner_inject_exchange_fault": (_I, [_P, _I]),
    "gw_expert_runner_reserve_prefill": (_I, [_P, _I32, _I32, _I32]),
    "gw_expert_apply": (_I, [_P, _P, _I, ctypes.POINTER(ExpertWeightsC), _P]),
    "gw_expert_apply_batch": (_I, [_P, _P, _I, _P, _P, _I32, _P]),
    "gw_expert_apply_assignments": (_I, [_P, _P, _I, _P, _I32, _P]),
    "gw_expert_apply_assignments_async": (_I, [_P, _P, _I, _P, _I32, _P]),
    "gw_moe_layer_forward": (_I, [_P, ctypes.POINTER(MoeLayerArgsC)]),
    "gw_moe_prefill_forward": (_I, [_P, ctypes.POINTER(MoeLayerArgsC)]),
    "gw_moe_prefill_forward_static": (_I, [_P, ctypes.POINTER(MoeLayerArgsC)]),
    "gw_expert_runner_prefill_view": (_I, [_P, ctypes.POINTER(PrefillViewC)]),
    "gw_moe_block_forward": (_I, [_P, ctypes.POINTER(MoeBlockArgsC)]),
    "gw_model_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "gw_model_close": (_I, [_P]),
    "gw_model_info_get": (_I, [_P, ctypes.POINTER(ModelInfoC)]),
    "gw_model_validate": (_I, [_P]),
    "gw_model_load_layer": (_I, [_P, _P, _I32, _P, ctypes.c_size_t]),
    "gw_model_load_expert": (_I, [_P, _P, _I32, _I32, _P]),
    "gw_graph_begin_capture": (_I, [_P]),
    "gw_graph_end_capture": (_I, [_P, ctypes.POINTER(_P)]),
    "gw_graph_launch": (_I, [_P]),
    "gw_graph_destroy": (_I, [_P]),
}


class GodwitError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python godwit_amd/build.py` "
            "(there is no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(status: int) -> None:
    if status != GW_OK:
        raise GodwitError(status, (lib.gw_last_error() or b"").decode())
