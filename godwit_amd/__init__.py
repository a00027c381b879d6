"""godwit_amd — MI355X-native MoE expert hot path of rayl15/Godwit.

Python mirror of the reference's engine API over the C ABI of
``libgodwit_hip.so`` (include/godwit_hip.h):

* :class:`Context` — MetalContext (Infrastructure/Metal/MetalContext.swift:36-179)
* :class:`ExpertLayout` — ExpertLayout (Install/InstallLayout.swift:14-121)
* :class:`ExpertRunner` with :class:`Weights` / :class:`Assignment` —
  ExpertRunner (Runtime/ExpertRunner.swift:10-363)
* :class:`Router` / :class:`Decision` — Router (Runtime/Router.swift:11-104)
* module functions ``mxfp4_dequant``, ``mxfp4_gemv``, ``mxfp4_gemv_bias``,
  ``expert_activation``, ``expert_accumulate`` — the Metal kernels'
  argument tables (Metal/Quant/*.metal, Metal/MoE/expert.metal).

Every call runs the HIP kernels; there is no CPU fallback.  Importing this
package fails when the library has not been built.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple, Union

import numpy as np

from ._lib import (ACT_GPTOSS_CLAMPED_GLU, ACT_SILU, BF16, F16, F32, SECTION_COUNT,
                   STATIC_SCRATCH_BYTES,
                   AssignmentC, ExpertLayoutC, ExpertWeightsC, GodwitError, ModelInfoC, MoeBlockArgsC, MoeLayerArgsC,
                   PrefillViewC,
                   check, lib)

__all__ = [
    "Context", "DeviceBuffer", "ExpertLayout", "ExpertRunner", "Weights", "Assignment",
    "Router", "Decision", "Graph", "GodwitError", "F32", "F16", "BF16", "SECTIONS",
    "mxfp4_dequant", "mxfp4_gemv", "mxfp4_gemv_bias", "expert_activation",
    "expert_accumulate", "device_count", "STATIC_SCRATCH_BYTES",
]

SECTIONS = ["gate_up_blocks", "gate_up_scales", "down_blocks", "down_scales",
            "gate_up_bias", "down_bias"]

ACTIVATIONS = {"gptOssClampedGLU": ACT_GPTOSS_CLAMPED_GLU, "silu": ACT_SILU}

_NP_DTYPES = {F32: np.float32, F16: np.float16, BF16: np.uint16}


def _dtype_of(arr: np.ndarray, dtype: Optional[int]) -> int:
    if dtype is not None:
        return dtype
    if arr.dtype == np.float32:
        return F32
    if arr.dtype == np.float16:
        return F16
    raise TypeError(f"pass dtype= for {arr.dtype} (bf16 data travels as uint16 bits)")


def device_count() -> int:
    n = ctypes.c_int(0)
    check(lib.gw_device_count(ctypes.byref(n)))
    return n.value


class DeviceBuffer:
    """A device allocation (MTLBuffer stand-in).  Freed by ``free`` or the context."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib.gw_malloc(ctx.handle, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value or 0

    def address(self, offset: int = 0) -> int:
        return self.ptr + int(offset)

    def upload(self, array, offset: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(array)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        check(lib.gw_memcpy_htod(self.ctx.handle, self.ptr + offset, a.ctypes.data, a.nbytes))
        return self

    def download(self, dtype, count: Optional[int] = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dt.itemsize
        out = np.empty(count, dt)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        check(lib.gw_memcpy_dtoh(self.ctx.handle, out.ctypes.data, self.ptr + offset,
                                 out.nbytes))
        return out

    def zero(self) -> "DeviceBuffer":
        check(lib.gw_memset_zero(self.ctx.handle, self.ptr, self.nbytes))
        return self

    def free(self) -> None:
        if self.ptr:
            check(lib.gw_free(self.ctx.handle, self.ptr))
            self.ptr = 0


class Context:
    """One HIP device and stream (MetalContext.init, MetalContext.swift:36-56)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        check(lib.gw_context_create(device, ctypes.byref(h)))
        self.handle = h.value
        self.device = device

    @property
    def cu_count(self) -> int:
        n = ctypes.c_int()
        check(lib.gw_context_cu_count(self.handle, ctypes.byref(n)))
        return n.value

    @property
    def stream(self) -> int:
        return lib.gw_context_stream(self.handle) or 0

    def synchronize(self) -> None:
        check(lib.gw_context_synchronize(self.handle))

    def buffer(self, array) -> DeviceBuffer:
        """MetalContext.buffer: a device copy of a host array."""
        a = np.ascontiguousarray(array)
        return DeviceBuffer(self, max(a.nbytes, 1)).upload(a)

    def empty(self, nbytes: int) -> DeviceBuffer:
        """MetalContext.emptyBuffer (contents undefined)."""
        return DeviceBuffer(self, max(int(nbytes), 1))

    def copy_async(self, dst: int, src: int, nbytes: int) -> None:
        """Enqueue a device-to-device copy on the context stream."""
        check(lib.gw_memcpy_dtod_async(self.handle, dst, src, nbytes))

    def fill_uniform_u8(self, buf: DeviceBuffer, lo: int, hi: int, seed: int,
                        offset: int = 0, count: Optional[int] = None, rows: int = 1,
                        row_stride: int = 0) -> None:
        """Seeded bytes uniform over [lo, hi]; with rows > 1, `rows` runs of `count`
        bytes starting row_stride bytes apart, in one launch."""
        n = buf.nbytes - offset if count is None else count
        if rows > 1:
            assert offset + (rows - 1) * row_stride + n <= buf.nbytes
        check(lib.gw_fill_uniform_u8(self.handle, buf.address(offset), n, rows, row_stride, lo,
                                     hi, seed))

    def fill_normal(self, buf: DeviceBuffer, dtype: int, count: int, mean: float, std: float,
                    seed: int, offset: int = 0, rows: int = 1, row_stride: int = 0) -> None:
        """Seeded normal(mean, std) values; rows as in fill_uniform_u8."""
        esz = 4 if dtype == F32 else 2
        assert offset + (rows - 1) * row_stride + count * esz <= buf.nbytes
        check(lib.gw_fill_normal(self.handle, buf.address(offset), dtype, count, rows, row_stride,
                                 mean, std, seed))

    # Profiler (Profiler.swift:11-98): per-kernel-family GPU time from hipEvents.
    def set_profiling(self, on: bool) -> None:
        check(lib.gw_context_set_profiling(self.handle, 1 if on else 0))

    def profile(self, name: str) -> Tuple[float, int]:
        ms = ctypes.c_double()
        n = ctypes.c_int64()
        check(lib.gw_context_profile_read(self.handle, name.encode(), ctypes.byref(ms),
                                          ctypes.byref(n)))
        return ms.value, n.value

    def profile_reset(self) -> None:
        check(lib.gw_context_profile_reset(self.handle))

    def close(self) -> None:
        if self.handle:
            check(lib.gw_context_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Graph:
    """A captured, replayable sequence of enqueue-only calls on one context."""

    def __init__(self, ctx: Context, handle):
        self.ctx = ctx
        self.handle = handle

    @staticmethod
    def capture(ctx: Context, body) -> "Graph":
        check(lib.gw_graph_begin_capture(ctx.handle))
        h = ctypes.c_void_p()
        try:
            body()
        except BaseException:
            # end the capture and drop the partial graph, then re-raise
            if lib.gw_graph_end_capture(ctx.handle, ctypes.byref(h)) == 0 and h.value:
                lib.gw_graph_destroy(h.value)
            raise
        check(lib.gw_graph_end_capture(ctx.handle, ctypes.byref(h)))
        return Graph(ctx, h.value)

    def launch(self) -> None:
        check(lib.gw_graph_launch(self.handle))

    def destroy(self) -> None:
        if self.handle:
            check(lib.gw_graph_destroy(self.handle))
            self.handle = None


class ExpertLayout:
    """Per-expert stride with six page-aligned sections (InstallLayout.swift:14-121)."""

    page_size = 16384

    def __init__(self, hidden_size: int, intermediate_size: int, expert_count: int):
        c = ExpertLayoutC()
        check(lib.gw_expert_layout_init(hidden_size, intermediate_size, expert_count,
                                        ctypes.byref(c)))
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.expert_count = expert_count
        self.offsets: Dict[str, int] = {s: int(c.offsets[i]) for i, s in enumerate(SECTIONS)}
        self.sizes: Dict[str, int] = {s: int(c.sizes[i]) for i, s in enumerate(SECTIONS)}
        self.stride = int(c.stride)

    def expert_offset(self, expert: int) -> int:
        if not 0 <= expert < self.expert_count:
            raise IndexError(f"expert {expert} out of range")
        return expert * self.stride

    def offset(self, expert: int, section: str) -> int:
        return self.expert_offset(expert) + self.offsets[section]

    def size(self, section: str) -> int:
        return self.sizes[section]

    @property
    def layer_file_size(self) -> int:
        return self.stride * self.expert_count

    @property
    def payload_per_expert(self) -> int:
        return sum(self.sizes.values())

    @property
    def padding_overhead(self) -> float:
        return 1.0 - self.payload_per_expert / self.stride

    def offsets_array(self):
        return [self.offsets[s] for s in SECTIONS]


SECTION_NAMES = ("gate_up_blocks", "gate_up_scales", "down_blocks", "down_scales",
                 "gate_up_bias", "down_bias")


class ModelReader:
    """A .gwt installation (ModelReader, Runtime/ModelReader.swift:11-111): the manifest's
    counts, stride, sections and the MoE spec fields, and its expert layer files read
    into device memory with unchanged bytes."""

    def __init__(self, directory: str):
        h = ctypes.c_void_p()
        check(lib.gw_model_open(os.fsencode(directory), ctypes.byref(h)))
        self.handle = h.value
        info = ModelInfoC()
        check(lib.gw_model_info_get(self.handle, ctypes.byref(info)))
        self.format_version = info.format_version
        self.layer_count = info.layer_count
        self.expert_count = info.expert_count
        self.expert_stride = info.expert_stride
        self.sections = {n: (info.section_offset[i], info.section_length[i])
                         for i, n in enumerate(SECTION_NAMES)}
        self.hidden_size = info.hidden_size
        self.intermediate_size = info.intermediate_size
        self.experts_per_token = info.experts_per_token
        self.rms_norm_epsilon = info.rms_norm_epsilon
        self.activation = ("gptOssClampedGLU", "silu")[info.activation]
        self.activation_limit = info.activation_limit
        self.activation_alpha = info.activation_alpha
        self.expert_bias = bool(info.expert_bias)
        self.router_bias = bool(info.router_bias)

    @property
    def layer_file_size(self) -> int:
        return self.expert_stride * self.expert_count

    def validate(self) -> None:
        """GodwitManifest.validate: every layer file has the size the manifest implies."""
        check(lib.gw_model_validate(self.handle))

    def load_layer(self, ctx: "Context", layer: int) -> "DeviceBuffer":
        """Layer `layer`'s expert file, resident on the device (the experts_base of
        layer_forward)."""
        buf = ctx.empty(self.layer_file_size)
        check(lib.gw_model_load_layer(ctx.handle, self.handle, layer, buf.ptr, buf.nbytes))
        return buf

    def load_expert(self, ctx: "Context", layer: int, expert: int) -> "DeviceBuffer":
        """One expert stride, all six sections (ModelReader.loadExpertStride)."""
        buf = ctx.empty(self.expert_stride)
        check(lib.gw_model_load_expert(ctx.handle, self.handle, layer, expert, buf.ptr))
        return buf

    def close(self) -> None:
        if self.handle:
            check(lib.gw_model_close(self.handle))
            self.handle = None


@dataclass
class Weights:
    """ExpertRunner.Weights (ExpertRunner.swift:54-64): one expert stride plus offsets."""
    buffer: Union[DeviceBuffer, int]
    offsets: Dict[str, int]

    def address(self) -> int:
        return self.buffer.ptr if isinstance(self.buffer, DeviceBuffer) else int(self.buffer)

    def c(self) -> ExpertWeightsC:
        w = ExpertWeightsC()
        w.buffer = self.address()
        for i, s in enumerate(SECTIONS):
            w.offsets[i] = int(self.offsets.get(s, 0))
        return w


@dataclass
class Assignment:
    """ExpertRunner.Assignment (ExpertRunner.swift:88-98)."""
    weights: Weights
    token: int
    routing_weight: float


class ExpertRunner:
    """Runs experts' feed-forward branch on the GPU (ExpertRunner.swift:10-363).

    ``apply`` / ``apply_batch`` take a host vector like the Swift methods and
    return host arrays; ``apply_assignments`` works on device buffers and
    accumulates in place.
    """

    def __init__(self, ctx: Context, hidden_size: int, intermediate_size: int,
                 activation: str = "gptOssClampedGLU", swiglu_limit: float = 7.0,
                 swiglu_alpha: float = 1.702, bias_dtype: int = BF16):
        self.ctx = ctx
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.activation = activation
        self.swiglu_limit = swiglu_limit
        self.swiglu_alpha = swiglu_alpha
        h = ctypes.c_void_p()
        check(lib.gw_expert_runner_create(ctx.handle, hidden_size, intermediate_size,
                                          ACTIVATIONS[activation], swiglu_limit, swiglu_alpha,
                                          ctypes.byref(h)))
        self.handle = h.value
        if bias_dtype != BF16:
            rc = lib.gw_expert_runner_set_bias_dtype(self.handle, bias_dtype)
            if rc != 0:
                err = GodwitError(rc, (lib.gw_last_error() or b"").decode())
                lib.gw_expert_runner_destroy(self.handle)
                self.handle = None
                raise err
        self._x: Optional[DeviceBuffer] = None
        self._y: Optional[DeviceBuffer] = None

    @property
    def section_offsets(self) -> Dict[str, int]:
        arr = (ctypes.c_int64 * SECTION_COUNT)()
        check(lib.gw_expert_runner_section_offsets(self.handle, arr))
        return {s: int(arr[i]) for i, s in enumerate(SECTIONS)}

    def _scratch(self, x: np.ndarray) -> Tuple[DeviceBuffer, DeviceBuffer]:
        need = max(x.nbytes, 4 * self.hidden_size)
        if self._x is None or self._x.nbytes < need:
            if self._x is not None:
                self._x.free()
            self._x = self.ctx.empty(need)
        if self._y is None:
            self._y = self.ctx.empty(4 * self.hidden_size)
        self._x.upload(x)
        return self._x, self._y

    def apply(self, input, weights: Weights, dtype: Optional[int] = None) -> np.ndarray:
        """ExpertRunner.apply (:275-331): the expert's output without routing weight."""
        x = np.ascontiguousarray(input)
        if x.size != self.hidden_size:
            raise ValueError(f"expected {self.hidden_size} inputs")
        dt = _dtype_of(x, dtype)
        xb, yb = self._scratch(x)
        w = weights.c()
        check(lib.gw_expert_apply(self.handle, xb.ptr, dt, ctypes.byref(w), yb.ptr))
        return yb.download(np.float32, self.hidden_size)

    def apply_batch(self, input, experts: Sequence[Tuple[Weights, float]],
                    dtype: Optional[int] = None) -> np.ndarray:
        """ExpertRunner.applyBatch (:191-269): sum of weighted expert outputs."""
        x = np.ascontiguousarray(input)
        if x.size != self.hidden_size:
            raise ValueError(f"expected {self.hidden_size} inputs")
        dt = _dtype_of(x, dtype)
        xb, yb = self._scratch(x)
        n = len(experts)
        ws = (ExpertWeightsC * max(n, 1))(*[w.c() for w, _ in experts])
        rw = np.array([float(r) for _, r in experts] or [0.0], np.float32)
        check(lib.gw_expert_apply_batch(self.handle, xb.ptr, dt, ws, rw.ctypes.data, n, yb.ptr))
        return yb.download(np.float32, self.hidden_size)

    def apply_assignments(self, inputs: DeviceBuffer, assignments: Sequence[Assignment],
                          outputs: DeviceBuffer, dtype: int = F16, wait: bool = True) -> None:
        """ExpertRunner.applyAssignments (:108-182): outputs[token] += w * expert(x)."""
        n = len(assignments)
        if n == 0:
            return
        arr = (AssignmentC * n)()
        for i, a in enumerate(assignments):
            arr[i].weights = a.weights.c()
            arr[i].token = int(a.token)
            arr[i].routing_weight = float(a.routing_weight)
        fn = lib.gw_expert_apply_assignments if wait else lib.gw_expert_apply_assignments_async
        check(fn(self.handle, inputs.ptr, dtype, arr, n, outputs.ptr))

    def layer_forward(self, experts_base: int, expert_stride: int, expert_count: int,
                      top_k: int, x: int, x_dtype: int, tokens: int, out: int,
                      logits: int = 0, router_weight: int = 0, router_weight_dtype: int = BF16,
                      router_bias: int = 0, router_bias_dtype: int = BF16, out_bf16: int = 0,
                      routing_ids: int = 0, routing_weights: int = 0) -> None:
        """MoE block of TransformerLayer.forward (TransformerLayer.swift:140-238), on the
        device; all pointer arguments are device addresses.  Enqueue only."""
        a = self._layer_args(experts_base, expert_stride, expert_count, top_k, x, x_dtype,
                             tokens, out, logits, router_weight, router_weight_dtype,
                             router_bias, router_bias_dtype, out_bf16, routing_ids,
                             routing_weights)
        check(lib.gw_moe_layer_forward(self.handle, ctypes.byref(a)))

    @staticmethod
    def _layer_args(experts_base, expert_stride, expert_count, top_k, x, x_dtype, tokens, out,
                    logits, router_weight, router_weight_dtype, router_bias, router_bias_dtype,
                    out_bf16, routing_ids, routing_weights):
        a = MoeLayerArgsC()
        a.experts_base = experts_base
        a.expert_stride = expert_stride
        a.expert_count = expert_count
        a.top_k = top_k
        a.logits = logits or None
        a.router_weight = router_weight or None
        a.router_weight_dtype = router_weight_dtype
        a.router_bias = router_bias or None
        a.router_bias_dtype = router_bias_dtype
        a.x = x
        a.x_dtype = x_dtype
        a.tokens = tokens
        a.out = out
        a.out_bf16 = out_bf16 or None
        a.routing_ids = routing_ids or None
        a.routing_weights = routing_weights or None
        return a

    def prefill_forward(self, experts_base: int, expert_stride: int, expert_count: int,
                        top_k: int, x: int, x_dtype: int, tokens: int, out: int,
                        logits: int = 0, router_weight: int = 0, router_weight_dtype: int = BF16,
                        router_bias: int = 0, router_bias_dtype: int = BF16, out_bf16: int = 0,
                        routing_ids: int = 0, routing_weights: int = 0) -> None:
        """Batched prefill of the MoE block (TransformerLayer.swift:140-238 with T > 1) as
        grouped GEMMs on the matrix cores; same arguments as layer_forward.  Enqueue only."""
        a = self._layer_args(experts_base, expert_stride, expert_count, top_k, x, x_dtype,
                             tokens, out, logits, router_weight, router_weight_dtype,
                             router_bias, router_bias_dtype, out_bf16, routing_ids,
                             routing_weights)
        check(lib.gw_moe_prefill_forward(self.handle, ctypes.byref(a)))

    def prefill_forward_static(self, experts_base: int, expert_stride: int, expert_count: int,
                               top_k: int, x: int, x_dtype: int, tokens: int, out: int,
                               logits: int = 0, router_weight: int = 0,
                               router_weight_dtype: int = BF16, router_bias: int = 0,
                               router_bias_dtype: int = BF16, out_bf16: int = 0,
                               routing_ids: int = 0, routing_weights: int = 0) -> None:
        """prefill_forward with its scratch in the library's fixed per-device array
        (STATIC_SCRATCH_BYTES) instead of the runner's buffer: allocates nothing.
        Calls that overlap on one device race.  Enqueue only."""
        a = self._layer_args(experts_base, expert_stride, expert_count, top_k, x, x_dtype,
                             tokens, out, logits, router_weight, router_weight_dtype,
                             router_bias, router_bias_dtype, out_bf16, routing_ids,
                             routing_weights)
        check(lib.gw_moe_prefill_forward_static(self.handle, ctypes.byref(a)))

    def block_forward(self, experts_base: int, expert_stride: int, expert_count: int,
                      top_k: int, tokens: int, stream: int, norm_weight: int,
                      epsilon: float, norm_weight_dtype: int = BF16, logits: int = 0,
                      router_weight: int = 0, router_weight_dtype: int = BF16,
                      router_bias: int = 0, router_bias_dtype: int = BF16,
                      out_bf16: int = 0, routing_ids: int = 0,
                      routing_weights: int = 0) -> None:
        """The MoE block with its surroundings (TransformerLayer.swift:140-143 and
        232-238): stream += MoE(RMSNorm(stream)), stream fp32 [tokens, hidden] updated in
        place; the router (when logits is 0) sees the normalised rows.  Enqueue only."""
        b = MoeBlockArgsC()
        b.layer = self._layer_args(experts_base, expert_stride, expert_count, top_k, 0, F16,
                                   tokens, 0, logits, router_weight, router_weight_dtype,
                                   router_bias, router_bias_dtype, out_bf16, routing_ids,
                                   routing_weights)
        b.stream = stream
        b.norm_weight = norm_weight
        b.norm_weight_dtype = norm_weight_dtype
        b.epsilon = epsilon
        check(lib.gw_moe_block_forward(self.handle, ctypes.byref(b)))

    def prefill_view(self) -> dict:
        """Device addresses of the last grouped batch's routing, fp16 activations
        ([tokens * top_k, intermediate]; activation_plane 0) and per-entry expert
        outputs in this runner's prefill scratch; valid until its next batch."""
        v = PrefillViewC()
        check(lib.gw_expert_runner_prefill_view(self.handle, ctypes.byref(v)))
        return {"routing_ids": v.routing_ids, "routing_weights": v.routing_weights,
                "activations": v.activations, "activation_plane": v.activation_plane,
                "expert_outputs": v.expert_outputs, "tokens": v.tokens, "top_k": v.top_k}

    def reserve_prefill(self, max_tokens: int, top_k: int, expert_count: int) -> None:
        """Sizes the prefill scratch up front (required before capturing a graph)."""
        check(lib.gw_expert_runner_reserve_prefill(self.handle, max_tokens, top_k, expert_count))

    def sync_errors(self) -> int:
        """Waves of the one-token layer kernel whose exchange wait gave up since
        creation (0 when every result is valid).  Waits for the runner's stream."""
        n = ctypes.c_uint32(0)
        check(lib.gw_expert_runner_sync_errors(self.handle, ctypes.byref(n)))
        return int(n.value)

    def set_wait_limit(self, polls: int) -> None:
        """Polls of the one-token layer's exchange before a wait gives up (0: default)."""
        check(lib.gw_expert_runner_set_wait_limit(self.handle, polls))

    def inject_exchange_fault(self, enable: bool) -> None:
        """Test hook: one-token layers read an exchange slot nobody writes, so every
        wait gives up (and every kernel still exits)."""
        check(lib.gw_expert_runner_inject_exchange_fault(self.handle, 1 if enable else 0))

    def close(self) -> None:
        for b in (self._x, self._y):
            if b is not None:
                b.free()
        self._x = self._y = None
        if self.handle:
            check(lib.gw_expert_runner_destroy(self.handle))
            self.handle = None


@dataclass
class Decision:
    """Router.Decision (Router.swift:13-23): ids highest logit first, softmax weights."""
    experts: List[int]
    weights: List[float] = field(default_factory=list)


class Router:
    """Router (Router.swift:11-104): logits on the GPU, selection on the host."""

    def __init__(self, ctx: Context, expert_count: int, hidden_size: int, top_k: int):
        self.ctx = ctx
        self.expert_count = expert_count
        self.hidden_size = hidden_size
        self.top_k = top_k

    def logits(self, hidden, weight: DeviceBuffer, bias: Optional[DeviceBuffer],
               weight_dtype: int = BF16, bias_dtype: int = BF16,
               dtype: Optional[int] = None) -> np.ndarray:
        x = np.ascontiguousarray(hidden)
        if x.size != self.hidden_size:
            raise ValueError(f"expected {self.hidden_size} inputs")
        dt = _dtype_of(x, dtype)
        xb = self.ctx.buffer(x)
        out = self.ctx.empty(4 * self.expert_count)
        try:
            check(lib.gw_router_logits(self.ctx.handle, weight.ptr, weight_dtype,
                                       bias.ptr if bias is not None else None, bias_dtype, xb.ptr,
                                       dt, out.ptr, self.expert_count, self.hidden_size, 1))
            return out.download(np.float32, self.expert_count)
        finally:
            xb.free()
            out.free()

    def select(self, logits) -> Decision:
        lg = np.ascontiguousarray(logits, np.float32)
        if lg.size != self.expert_count:
            raise ValueError(f"expected {self.expert_count} logits")
        ids = np.empty(self.top_k, np.int32)
        w = np.empty(self.top_k, np.float32)
        check(lib.gw_router_select(lg.ctypes.data, lg.size, self.top_k, ids.ctypes.data,
                                   w.ctypes.data))
        return Decision([int(i) for i in ids], [float(v) for v in w])

    def route(self, hidden, weight: DeviceBuffer, bias: Optional[DeviceBuffer], **kw) -> Decision:
        return self.select(self.logits(hidden, weight, bias, **kw))


# ---- kernel-level entry points -----------------------------------------------

def mxfp4_dequant(ctx: Context, packed: DeviceBuffer, scales: DeviceBuffer, blocks: int,
                  out: DeviceBuffer) -> None:
    check(lib.gw_mxfp4_dequant(ctx.handle, packed.ptr, scales.ptr, blocks, out.ptr))


def mxfp4_gemv(ctx: Context, packed: DeviceBuffer, scales: DeviceBuffer, x: DeviceBuffer,
               x_dtype: int, y: DeviceBuffer, rows: int, cols: int) -> None:
    check(lib.gw_mxfp4_gemv(ctx.handle, packed.ptr, scales.ptr, x.ptr, x_dtype, y.ptr, rows,
                            cols))


def mxfp4_gemv_bias(ctx: Context, packed: DeviceBuffer, scales: DeviceBuffer,
                    bias: Optional[DeviceBuffer], bias_dtype: int, x: DeviceBuffer,
                    x_dtype: int, y: DeviceBuffer, rows: int, cols: int) -> None:
    check(lib.gw_mxfp4_gemv_bias(ctx.handle, packed.ptr, scales.ptr,
                                 bias.ptr if bias is not None else None, bias_dtype, x.ptr,
                                 x_dtype, y.ptr, rows, cols))


def expert_activation(ctx: Context, kind: str, gate_up: DeviceBuffer, out: DeviceBuffer,
                      width: int, limit: float = 7.0, alpha: float = 1.702) -> None:
    check(lib.gw_expert_activation(ctx.handle, ACTIVATIONS[kind], gate_up.ptr, out.ptr, width,
                                   limit, alpha))


def expert_accumulate(ctx: Context, expert_out: DeviceBuffer, dst: DeviceBuffer, weight: float,
                      width: int) -> None:
    check(lib.gw_expert_accumulate(ctx.handle, expert_out.ptr, dst.ptr, weight, width))
