"""CPU oracle for the MXFP4 MoE expert hot path — TEST INFRASTRUCTURE ONLY.

A ctypes binding of ``oracle/libgodwit_oracle.so``, the C restatement of the
reference's CPU ground truth (``godwit_oracle.c`` cites the reference line each
function follows).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this package; the product
(``godwit_amd``) never does, and fails loudly if its HIP library is missing.

All arrays are numpy; inputs are converted to contiguous arrays of the dtype
the C function expects.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgodwit_oracle.so")

ACT_GPTOSS = 0
ACT_SWIGLU = 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float


def build() -> None:
    """Compile the oracle with its Makefile (gcc -O2 -ffp-contract=off)."""
    subprocess.check_call(["make", "-s", "-C", _HERE])


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    sig = {
        "gwo_f32_to_f16": (ctypes.c_uint16, [_F]),
        "gwo_f16_to_f32": (_F, [ctypes.c_uint16]),
        "gwo_f32_to_bf16": (ctypes.c_uint16, [_F]),
        "gwo_bf16_to_f32": (_F, [ctypes.c_uint16]),
        "gwo_codebook": (_F, [ctypes.c_int]),
        "gwo_decode_scale": (_F, [ctypes.c_uint8]),
        "gwo_decode_block": (None, [_P, ctypes.c_uint8, _P]),
        "gwo_decode": (None, [_P, _P, _I64, _P]),
        "gwo_scale_byte_for_peak": (ctypes.c_uint8, [_F]),
        "gwo_code_for_magnitude": (ctypes.c_uint8, [_F]),
        "gwo_encode_block": (ctypes.c_uint8, [_P, ctypes.c_int, _P]),
        "gwo_encode": (None, [_P, _I64, _P, _P]),
        "gwo_reference_mxfp4": (None, [_P, _P, _P, _P, _I64, _I64]),
        "gwo_gemv_bias": (None, [_P, _P, _P, _P, _P, _I64, _I64]),
        "gwo_set_threads": (None, [ctypes.c_int]),
        "gwo_gptoss_activation_f32": (_F, [_F, _F, _F, _F]),
        "gwo_swiglu_f32": (_F, [_F, _F]),
        "gwo_activation": (None, [ctypes.c_int, _P, _P, _I64, _F, _F]),
        "gwo_accumulate": (None, [_P, _P, _F, _I64]),
        "gwo_rmsnorm_f16": (None, [_P, _P, _I64, _F, _P]),
        "gwo_residual_add": (None, [_P, _P, _I64]),
        "gwo_router_logits": (None, [_P, _P, _P, _P, _I64, _I64]),
        "gwo_router_select": (None, [_P, _I64, _I64, _P, _P]),
        "gwo_expert_apply": (None, [_P, _P, _P, _I64, _I64, ctypes.c_int, _F, _F]),
        "gwo_expert_apply_batch": (None, [_P, _P, _I32, _P, _P, _I64, _I64, ctypes.c_int, _F, _F]),
        "gwo_apply_assignments": (None, [_P, _P, _I32, _P, _P, _I64, _I64, ctypes.c_int, _F, _F]),
        "gwo_moe_layer": (None, [_P, _I64, _I64, _P, _P, _I32, _P, _P, _P, _I64, _I64,
                                 ctypes.c_int, _F, _F]),
        "gwo_xorshift_bytes": (None, [ctypes.c_uint32, _P, _I64]),
        "gwo_xorshift_activations_f16": (None, [ctypes.c_uint32, _P, _I64]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = _load()


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


# ---- number formats ------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    return np.array([_lib.gwo_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def f32_to_bf16_bits(x) -> np.ndarray:
    """BFloat16.fromFloat (RNE, NaN kept), vectorised with the same bit recipe."""
    bits = _c(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    rounding = ((bits >> 16) & 1) + 0x7FFF
    out = ((bits + rounding) >> 16).astype(np.uint16)
    out[nan] = ((bits[nan] >> 16) | 0x0040).astype(np.uint16)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    return (_c(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to_bf16(x) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ---- codec ---------------------------------------------------------------

def decode_scale(byte: int) -> float:
    return _lib.gwo_decode_scale(int(byte))


def decode(packed, scales, blocks: int) -> np.ndarray:
    p, s = _c(packed, np.uint8), _c(scales, np.uint8)
    assert p.size >= blocks * 16 and s.size >= blocks
    out = np.empty(blocks * 32, np.float32)
    _lib.gwo_decode(_ptr(p), _ptr(s), blocks, _ptr(out))
    return out


def scale_byte_for_peak(peak: float) -> int:
    return int(_lib.gwo_scale_byte_for_peak(float(peak)))


def code_for_magnitude(v: float) -> int:
    return int(_lib.gwo_code_for_magnitude(float(v)))


def encode(weights):
    w = _c(weights, np.float32).ravel()
    blocks = (w.size + 31) // 32
    packed = np.empty(blocks * 16, np.uint8)
    scales = np.empty(blocks, np.uint8)
    _lib.gwo_encode(_ptr(w), w.size, _ptr(packed), _ptr(scales))
    return packed, scales


# ---- GEMV / activations --------------------------------------------------

def reference_mxfp4(packed, scales, x, rows: int, cols: int) -> np.ndarray:
    p, s, xv = _c(packed, np.uint8), _c(scales, np.uint8), _c(x, np.float32)
    assert p.size == rows * cols // 2 and s.size == rows * cols // 32 and xv.size == cols
    y = np.empty(rows, np.float32)
    _lib.gwo_reference_mxfp4(_ptr(p), _ptr(s), _ptr(xv), _ptr(y), rows, cols)
    return y


def set_threads(threads: int) -> None:
    """Row-parallel GEMVs on `threads` host threads (1: serial); same results."""
    _lib.gwo_set_threads(int(threads))


def gemv_bias(packed, scales, bias, x, rows: int, cols: int) -> np.ndarray:
    p, s, xv = _c(packed, np.uint8), _c(scales, np.uint8), _c(x, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    assert p.size == rows * cols // 2 and s.size == rows * cols // 32 and xv.size == cols
    y = np.empty(rows, np.float32)
    _lib.gwo_gemv_bias(_ptr(p), _ptr(s), _ptr(b), _ptr(xv), _ptr(y), rows, cols)
    return y


def gptoss_activation(gate: float, up: float, limit=7.0, alpha=1.702) -> float:
    return _lib.gwo_gptoss_activation_f32(gate, up, limit, alpha)


def swiglu(gate: float, up: float) -> float:
    return _lib.gwo_swiglu_f32(gate, up)


def activation(kind: int, gate_up, limit=7.0, alpha=1.702) -> np.ndarray:
    """Interleaved fp32 gate_up [2F] -> fp16 [F] (returned as np.float16)."""
    gu = _c(gate_up, np.float32)
    width = gu.size // 2
    out = np.empty(width, np.uint16)
    _lib.gwo_activation(kind, _ptr(gu), _ptr(out), width, limit, alpha)
    return out.view(np.float16)


def accumulate(expert_out, dst, weight: float) -> np.ndarray:
    o, d = _c(expert_out, np.float32), _c(dst, np.float32).copy()
    _lib.gwo_accumulate(_ptr(o), _ptr(d), weight, o.size)
    return d


def rmsnorm_f16(x, weight_bf16, eps: float) -> np.ndarray:
    """fp16 bits of RMSNorm(x) per row of a [T, width] fp32 array (bf16 weight bits)."""
    x = _c(np.atleast_2d(x), np.float32)
    w = _c(weight_bf16, np.uint16)
    out = np.empty(x.shape, np.uint16)
    for t in range(x.shape[0]):
        _lib.gwo_rmsnorm_f16(_ptr(x[t]), _ptr(w), x.shape[1], eps, _ptr(out[t]))
    return out


def residual_add(stream, combined) -> np.ndarray:
    s, c = _c(stream, np.float32).copy(), _c(combined, np.float32)
    _lib.gwo_residual_add(_ptr(s), _ptr(c), s.size)
    return s


def router_logits(weight, bias, x, experts: int, hidden: int) -> np.ndarray:
    w, xv = _c(weight, np.float32), _c(x, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    out = np.empty(experts, np.float32)
    _lib.gwo_router_logits(_ptr(w), _ptr(b), _ptr(xv), _ptr(out), experts, hidden)
    return out


def router_select(logits, top_k: int):
    lg = _c(logits, np.float32)
    ids = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    _lib.gwo_router_select(_ptr(lg), lg.size, top_k, _ptr(ids), _ptr(w))
    return ids, w


# ---- expert composition --------------------------------------------------

class _Expert(ctypes.Structure):
    _fields_ = [("gate_up_blocks", _P), ("gate_up_scales", _P), ("down_blocks", _P),
                ("down_scales", _P), ("gate_up_bias", _P), ("down_bias", _P)]


class _Assignment(ctypes.Structure):
    _fields_ = [("expert", _I32), ("token", _I32), ("weight", _F)]


class Expert:
    """One expert's six sections as numpy arrays (biases widened to fp32 or None)."""

    def __init__(self, gate_up_blocks, gate_up_scales, down_blocks, down_scales,
                 gate_up_bias=None, down_bias=None):
        self.arrays = [_c(gate_up_blocks, np.uint8), _c(gate_up_scales, np.uint8),
                       _c(down_blocks, np.uint8), _c(down_scales, np.uint8),
                       None if gate_up_bias is None else _c(gate_up_bias, np.float32),
                       None if down_bias is None else _c(down_bias, np.float32)]

    def struct(self) -> _Expert:
        return _Expert(*[_ptr(a) for a in self.arrays])


def _experts_array(experts):
    arr = (_Expert * len(experts))(*[e.struct() for e in experts])
    return arr


def expert_apply(expert: Expert, x, hidden: int, inter: int, act=ACT_GPTOSS,
                 limit=7.0, alpha=1.702) -> np.ndarray:
    xv = _c(x, np.float32)
    out = np.empty(hidden, np.float32)
    s = expert.struct()
    _lib.gwo_expert_apply(ctypes.byref(s), _ptr(xv), _ptr(out), hidden, inter, act, limit, alpha)
    return out


def expert_apply_batch(experts, routing, x, hidden: int, inter: int, act=ACT_GPTOSS,
                       limit=7.0, alpha=1.702) -> np.ndarray:
    arr = _experts_array(experts)
    r = _c(routing, np.float32)
    xv = _c(x, np.float32)
    out = np.empty(hidden, np.float32)
    _lib.gwo_expert_apply_batch(arr, _ptr(r), len(experts), _ptr(xv), _ptr(out), hidden, inter,
                                act, limit, alpha)
    return out


def apply_assignments(experts, assignments, inputs, outputs, hidden: int, inter: int,
                      act=ACT_GPTOSS, limit=7.0, alpha=1.702) -> np.ndarray:
    """assignments: list of (expert_index, token, weight).  Returns updated outputs."""
    arr = _experts_array(experts)
    a = (_Assignment * len(assignments))(*[_Assignment(int(e), int(t), float(w))
                                           for e, t, w in assignments])
    inp = _c(inputs, np.float32)
    out = _c(outputs, np.float32).copy()
    _lib.gwo_apply_assignments(arr, a, len(assignments), _ptr(inp), _ptr(out), hidden, inter,
                               act, limit, alpha)
    return out


def moe_layer(experts, top_k: int, logits, x, hidden: int, inter: int, act=ACT_GPTOSS,
              limit=7.0, alpha=1.702):
    """Returns (out [T, H], ids [T, k], weights [T, k])."""
    arr = _experts_array(experts)
    lg = _c(logits, np.float32)
    xv = _c(x, np.float32)
    tokens = xv.size // hidden
    out = np.empty((tokens, hidden), np.float32)
    ids = np.empty((tokens, top_k), np.int32)
    w = np.empty((tokens, top_k), np.float32)
    _lib.gwo_moe_layer(arr, len(experts), top_k, _ptr(lg), _ptr(xv), tokens, _ptr(out),
                       _ptr(ids), _ptr(w), hidden, inter, act, limit, alpha)
    return out, ids, w


# ---- deterministic inputs ------------------------------------------------

def xorshift_bytes(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint8)
    _lib.gwo_xorshift_bytes(seed, _ptr(out), count)
    return out


def xorshift_activations_f16(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint16)
    _lib.gwo_xorshift_activations_f16(seed, _ptr(out), count)
    return out.view(np.float16)
