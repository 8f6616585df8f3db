"""Host-side mirror of the reference crate's public executor API over the gfx950 C ABI.

Each class mirrors one reference type (cited) with the same method names, argument meaning
and error behaviour (``FlatHipError.variant`` names the reference error variant). Device
memory is plain HIP memory owned by :class:`DeviceBuffer`; nothing here computes attention on
the host.
"""

from __future__ import annotations

import contextlib
import ctypes
import types
import weakref
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib as L
from ._lib import check, lib

# ----------------------------------------------------------------------------- value types


@dataclass(frozen=True)
class AttentionShape:
    """AttentionShape src/lib.rs:212."""
    batch: int
    heads: int
    seq_len: int
    head_dim: int

    def tensor_len(self):
        return self.batch * self.heads * self.seq_len * self.head_dim

    def lse_len(self):
        return self.batch * self.heads * self.seq_len

    def c(self):
        return L.AttentionShapeC(self.batch, self.heads, self.seq_len, self.head_dim)


@dataclass(frozen=True)
class GroupedAttentionShape:
    """GroupedAttentionShape src/grouped.rs:18."""
    batch: int
    q_heads: int
    kv_heads: int
    seq_len: int
    head_dim: int

    def q_tensor_len(self):
        return self.batch * self.q_heads * self.seq_len * self.head_dim

    def kv_tensor_len(self):
        return self.batch * self.kv_heads * self.seq_len * self.head_dim

    def lse_len(self):
        return self.batch * self.q_heads * self.seq_len

    def c(self):
        return L.GroupedShapeC(self.batch, self.q_heads, self.kv_heads, self.seq_len,
                               self.head_dim)


@dataclass(frozen=True)
class AsymmetricGroupedAttentionShape:
    """AsymmetricGroupedAttentionShape src/asymmetric_grouped.rs:27."""
    batch: int
    q_heads: int
    kv_heads: int
    query_len: int
    kv_len: int
    head_dim: int
    query_position_offset: int = 0

    def q_tensor_len(self):
        return self.batch * self.q_heads * self.query_len * self.head_dim

    def kv_tensor_len(self):
        return self.batch * self.kv_heads * self.kv_len * self.head_dim

    def lse_len(self):
        return self.batch * self.q_heads * self.query_len

    def c(self):
        return L.AsymmetricShapeC(self.batch, self.q_heads, self.kv_heads, self.query_len,
                                  self.kv_len, self.head_dim, self.query_position_offset)


@dataclass(frozen=True)
class FlatAttentionConfig:
    """FlatAttentionConfig src/lib.rs:249."""
    causal: bool = False
    softmax_scale: Optional[float] = None

    def c(self):
        return L.ConfigC(int(self.causal), int(self.softmax_scale is not None),
                         float(self.softmax_scale or 0.0))

    def resolved_scale(self, head_dim: int) -> float:
        out = L.F32()
        check(lib().fa_resolved_scale(ctypes.byref(self.c()), head_dim, ctypes.byref(out)))
        return out.value


@dataclass(frozen=True)
class RotaryEmbeddingConfig:
    """RotaryEmbeddingConfig src/rotary_grouped.rs:14."""
    theta: float
    position_offset: int = 0

    def c(self):
        return L.RotaryC(self.theta, self.position_offset)


@dataclass(frozen=True)
class AsymmetricRotaryEmbeddingConfig:
    """AsymmetricRotaryEmbeddingConfig src/projection_asymmetric.rs:19."""
    theta: float
    query_position_offset: int = 0
    kv_position_offset: int = 0

    def c(self):
        return L.AsymmetricRotaryC(self.theta, self.query_position_offset,
                                   self.kv_position_offset)


@dataclass
class FlatAttentionOutput:
    """FlatAttentionOutput src/lib.rs:355 (output in the I/O dtype as stored, LSE f32)."""
    output: np.ndarray
    lse: np.ndarray


@dataclass(frozen=True)
class PackedLayout:
    """[O | LSE] geometry (PagedDecodeLayout src/wgpu_paged_decode.rs:18)."""
    output_elements: int
    lse_elements: int
    output_bytes: int
    lse_byte_offset: int
    combined_bytes: int


@dataclass(frozen=True)
class RuntimeDispatchTelemetry:
    """RuntimeDispatchTelemetry src/runtime_telemetry.rs:159."""
    kernel_id: str
    kernel_name: str
    query_rows: int
    kv_rows: int
    workgroups: tuple
    workgroup_size: int
    dispatch_count: int
    temporary_allocation_count: int
    temporary_allocation_bytes: int
    splits: int
    fallback_reason: Optional[str]
    device_name: str
    device_arch: str
    device_fingerprint: int


def packed_layout(output_elements: int, lse_elements: int, dtype: int) -> PackedLayout:
    c = L.PackedLayoutC()
    check(lib().fa_packed_layout_for(output_elements, lse_elements, dtype, ctypes.byref(c)))
    return PackedLayout(c.output_elements, c.lse_elements, c.output_bytes, c.lse_byte_offset,
                        c.combined_bytes)


# ----------------------------------------------------------------------------- dtypes

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bfloat16 bit patterns (uint16)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32)
    nan = (b & 0x7F800000) == 0x7F800000
    nan &= (b & 0x007FFFFF) != 0
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((b[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def host_storage(x: np.ndarray, dtype: int) -> np.ndarray:
    """f32 array -> storage array of `dtype` (f32, f16 as float16, bf16 as uint16 bits)."""
    if dtype == L.DTYPE_F32:
        return np.ascontiguousarray(x, np.float32)
    if dtype == L.DTYPE_F16:
        return np.ascontiguousarray(x, np.float32).astype(np.float16)
    return f32_to_bf16_bits(x)


def storage_to_f32(x: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == L.DTYPE_F32:
        return np.asarray(x, np.float32)
    if dtype == L.DTYPE_F16:
        return np.asarray(x).view(np.float16).astype(np.float32)
    return bf16_bits_to_f32(np.asarray(x).view(np.uint16))


def storage_np_dtype(dtype: int):
    return {L.DTYPE_F32: np.float32, L.DTYPE_F16: np.float16, L.DTYPE_BF16: np.uint16}[dtype]


# ----------------------------------------------------------------------------- context

class HipContext:
    """One device + one HIP stream (the owned-context half of WgpuFlatAttention
    src/wgpu_backend.rs:157-207)."""

    def __init__(self, device: int = 0):
        h = L.VP()
        check(lib().fa_ctx_create(device, ctypes.byref(h)))
        self.handle = h.value
        self._children = weakref.WeakSet()

    def _adopt(self, obj):
        """Track a dependent object so close() releases it before the context."""
        self._children.add(obj)

    def close(self):
        if getattr(self, "handle", None):
            for child in list(self._children):
                child.release()
            lib().fa_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return lib().fa_ctx_stream(self.handle)

    def synchronize(self):
        check(lib().fa_ctx_synchronize(self.handle))

    def capture_begin(self):
        """Start recording this context's launches into a HIP graph (fa_graph_capture_begin)."""
        check(lib().fa_graph_capture_begin(self.handle))

    def capture_end(self) -> "HipGraph":
        h = L.VP()
        check(lib().fa_graph_capture_end(self.handle, ctypes.byref(h)))
        return HipGraph(self, h.value)

    @contextlib.contextmanager
    def capture(self):
        """``with ctx.capture() as cap: <launches>`` then ``cap.graph.launch()``. The capture is
        ended (and its graph built) even when the body raises."""
        cap = types.SimpleNamespace(graph=None)
        self.capture_begin()
        try:
            yield cap
        finally:
            cap.graph = self.capture_end()

    def adapter_name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        check(lib().fa_ctx_device_name(self.handle, buf, 256))
        return buf.value.decode()

    def set_prefill_policy(self, prerotate_k: int):
        check(lib().fa_ctx_set_prefill_policy(self.handle, prerotate_k))

    def set_prefill_kernel(self, assembly: int):
        """-1 (default) and 1: the assembly main loop fa_prefill_a64_bf16 / _f16 where it
        applies (bf16 or f16, head_dim 128, RoPE with pre-rotated K, power-of-two GQA group);
        0: the HIP prefill kernels only."""
        check(lib().fa_ctx_set_prefill_kernel(self.handle, assembly))

    def set_decode_policy(self, grouped: int):
        """-1 automatic decode work layout (head-grouped workgroups where they apply), 0 one-wave
        workgroups; read when a PagedDecodePlan is prepared."""
        check(lib().fa_ctx_set_decode_policy(self.handle, grouped))

    def set_backward_policy(self, store_ds: int):
        """-1 automatic (16-bit storage: bwd_dkdv stores dS and dQ = dS K reads it back when the
        workspace fits in 2 GiB), 0 dQ recomputes S and dP."""
        check(lib().fa_ctx_set_backward_policy(self.handle, store_ds))

    def set_backward_kernel(self, assembly: int):
        """-1 (default) and 1: the assembly dK/dV kernel fa_bwd_dkdv_a64_bf16 where it applies
        (bf16, head_dim 128, seq_len a multiple of 128, dS stored); 0: the HIP kernel only."""
        check(lib().fa_ctx_set_backward_kernel(self.handle, assembly))

    def set_prefill_precision(self, mode: int):
        """0: rotated Q/K rounded to the 16-bit storage type before Q.K^T (default, fastest);
        1: split high/residual operands, f32-level scores for the 16-bit RoPE prefill."""
        check(lib().fa_ctx_set_prefill_precision(self.handle, mode))

    def set_kernel_timing(self, enable: bool):
        """Bracket every dispatch with HIP events on the context's stream (clears totals)."""
        check(lib().fa_ctx_set_kernel_timing(self.handle, 1 if enable else 0))

    def pause_kernel_timing(self, paused: bool):
        """Stop (or resume) bracketing dispatches with events, keeping the totals; never waits."""
        check(lib().fa_ctx_pause_kernel_timing(self.handle, 1 if paused else 0))

    def kernel_timing(self, kernel_id) -> tuple[float, int]:
        """(total ms, dispatch count) of one kernel since timing was enabled. `kernel_id` is an
        fa_kernel_id number or its name (e.g. "DecodePagedMfma")."""
        if isinstance(kernel_id, str):
            kernel_id = {v: k for k, v in L.KERNEL_IDS.items()}[kernel_id]
        ms, n = ctypes.c_double(), ctypes.c_uint64()
        check(lib().fa_ctx_kernel_timing(self.handle, kernel_id, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    def kernel_timing_range(self, kernel_id) -> tuple[float, float]:
        """(shortest, longest) single dispatch in ms of one kernel since timing was enabled."""
        if isinstance(kernel_id, str):
            kernel_id = {v: k for k, v in L.KERNEL_IDS.items()}[kernel_id]
        lo, hi = ctypes.c_double(), ctypes.c_double()
        check(lib().fa_ctx_kernel_timing_range(self.handle, kernel_id, ctypes.byref(lo),
                                               ctypes.byref(hi)))
        return lo.value, hi.value

    def last_telemetry(self) -> RuntimeDispatchTelemetry:
        t = L.TelemetryC()
        check(lib().fa_last_telemetry(self.handle, ctypes.byref(t)))
        return _telemetry(t)

    def forward_telemetry(self, shape, config: "FlatAttentionConfig" = None,
                          rotary: "RotaryEmbeddingConfig" = None,
                          dtype: int = L.DTYPE_F32) -> RuntimeDispatchTelemetry:
        """Passive snapshot of what a one-shot forward of `shape` (AttentionShape: MHA;
        GroupedAttentionShape: GQA, optional RoPE) would dispatch; no device work."""
        t = L.TelemetryC()
        cfg = ctypes.byref((config or FlatAttentionConfig()).c())
        if isinstance(shape, AttentionShape):
            check(lib().fa_forward_mha_telemetry(self.handle, ctypes.byref(shape.c()), cfg, dtype,
                                                 ctypes.byref(t)))
        else:
            rot = ctypes.byref(rotary.c()) if rotary is not None else None
            check(lib().fa_forward_gqa_rope_telemetry(self.handle, ctypes.byref(shape.c()), cfg,
                                                      rot, dtype, ctypes.byref(t)))
        return _telemetry(t)

    def kernel_variant_for_shape(self, head_dim: int, rope: bool, dtype: int) -> str:
        out = L.I32()
        check(lib().fa_kernel_variant_for_shape(self.handle, head_dim, int(rope), dtype,
                                                ctypes.byref(out)))
        return L.KERNEL_IDS[out.value]


def _telemetry(t) -> RuntimeDispatchTelemetry:
    return RuntimeDispatchTelemetry(
            L.KERNEL_IDS.get(t.kernel_id, str(t.kernel_id)), t.kernel_name.decode(), t.query_rows,
            t.kv_rows, tuple(t.workgroups), t.workgroup_size, t.dispatch_count,
            t.temporary_allocation_count, t.temporary_allocation_bytes, t.splits,
            t.fallback_reason.decode() if t.has_fallback_reason else None,
            t.device_name.decode(), t.device_arch.decode(), t.device_fingerprint)


class HipGraph:
    """An executable graph of captured launches (fa_graph_*): replays them on the context's
    stream with the buffers and arguments they were captured with."""

    def __init__(self, ctx: "HipContext", handle: int):
        self.ctx, self.handle = ctx, handle
        ctx._adopt(self)

    def launch(self):
        check(lib().fa_graph_launch(self.ctx.handle, self.handle))

    def release(self):
        if getattr(self, "handle", None):
            lib().fa_graph_destroy(self.handle)
        self.handle = None

    def __del__(self):
        self.release()


class DeviceBuffer:
    """Resident device buffer (WgpuResidentBuffer src/wgpu_backend.rs:112): pointer, byte size
    and the owning context. ``ptr`` may also wrap foreign memory (e.g. a torch tensor)."""

    def __init__(self, ctx: HipContext, nbytes: int, ptr: Optional[int] = None,
                 owned: bool = True):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        self.owned = owned and ptr is None
        if ptr is None:
            h = L.VP()
            check(lib().fa_buf_alloc(ctx.handle, self.nbytes, ctypes.byref(h)))
            ptr = h.value
        self.ptr = ptr
        ctx._adopt(self)

    @classmethod
    def from_array(cls, ctx: HipContext, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(ctx, arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray, offset: int = 0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        check(lib().fa_buf_upload(self.ctx.handle, self.ptr + offset, arr.ctypes.data,
                                  arr.nbytes))

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib().fa_buf_download(self.ctx.handle, out.ctypes.data, self.ptr + offset,
                                    out.nbytes))
        return out

    def fill_u32(self, value: int):
        check(lib().fa_buf_fill_u32(self.ctx.handle, self.ptr, value, self.nbytes // 4))

    def free(self):
        if self.owned and self.ptr and self.ctx.handle:
            lib().fa_buf_free(self.ctx.handle, self.ptr)
        self.ptr = 0

    release = free

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def download_attention(buf: DeviceBuffer, layout: PackedLayout, dtype: int) -> FlatAttentionOutput:
    """download_attention src/wgpu_backend.rs:588: read back the packed [O|LSE] buffer."""
    out = buf.download(storage_np_dtype(dtype), layout.output_elements)
    lse = buf.download(np.float32, layout.lse_elements, layout.lse_byte_offset)
    return FlatAttentionOutput(out, lse)


# ----------------------------------------------------------------------------- executors

class HipFlatAttention:
    """WgpuFlatAttention src/wgpu_backend.rs:157 (MHA, [B,H,S,D], packed [O|LSE])."""

    def __init__(self, ctx: Optional[HipContext] = None, dtype: int = L.DTYPE_F32):
        self.ctx = ctx or HipContext()
        self.dtype = dtype

    def adapter_name(self):
        return self.ctx.adapter_name()

    def kernel_variant_for_head_dim(self, head_dim: int) -> str:
        return self.ctx.kernel_variant_for_shape(head_dim, False, self.dtype)

    def upload(self, data: np.ndarray) -> DeviceBuffer:
        return DeviceBuffer.from_array(self.ctx, host_storage(data, self.dtype)
                                       if data.dtype == np.float32 else data)

    def layout(self, shape: AttentionShape) -> PackedLayout:
        return packed_layout(shape.tensor_len(), shape.lse_len(), self.dtype)

    def forward_resident(self, q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer,
                         shape: AttentionShape, config: FlatAttentionConfig,
                         out: Optional[DeviceBuffer] = None) -> DeviceBuffer:
        lay = self.layout(shape)
        out = out or DeviceBuffer(self.ctx, lay.combined_bytes)
        n = min(q.nbytes, k.nbytes, v.nbytes)
        check(lib().fa_forward_mha(self.ctx.handle, q.ptr, k.ptr, v.ptr, n, out.ptr, out.nbytes,
                                   ctypes.byref(shape.c()), ctypes.byref(config.c()),
                                   self.dtype))
        return out

    def download_attention(self, out: DeviceBuffer, shape: AttentionShape) -> FlatAttentionOutput:
        return download_attention(out, self.layout(shape), self.dtype)

    def forward(self, q: np.ndarray, k: np.ndarray, v: np.ndarray, shape: AttentionShape,
                config: FlatAttentionConfig) -> FlatAttentionOutput:
        qs, ks, vs = (host_storage(x, self.dtype) for x in (q, k, v))
        out = np.empty(shape.tensor_len(), storage_np_dtype(self.dtype))
        lse = np.empty(shape.lse_len(), np.float32)
        check(lib().fa_forward_mha_host(self.ctx.handle, qs.ctypes.data, ks.ctypes.data,
                                        vs.ctypes.data, qs.size, ks.size, vs.size,
                                        ctypes.byref(shape.c()), ctypes.byref(config.c()),
                                        self.dtype, out.ctypes.data, lse.ctypes.data))
        return FlatAttentionOutput(out, lse)

    def runtime_telemetry(self, shape: Optional[AttentionShape] = None,
                          config: Optional[FlatAttentionConfig] = None) -> RuntimeDispatchTelemetry:
        """runtime_telemetry src/wgpu_backend.rs: with a shape, the passive snapshot of the
        dispatch a forward of it would make (no device work); without, the last dispatch's."""
        if shape is None:
            return self.ctx.last_telemetry()
        return self.ctx.forward_telemetry(shape, config, None, self.dtype)


class HipRotaryGroupedAttention:
    """WgpuRotaryGroupedAttention src/wgpu_rotary_grouped_backend.rs:60 (GQA + fused RoPE)."""

    def __init__(self, ctx: Optional[HipContext] = None, dtype: int = L.DTYPE_F32):
        self.ctx = ctx or HipContext()
        self.dtype = dtype

    def upload(self, data: np.ndarray) -> DeviceBuffer:
        return DeviceBuffer.from_array(self.ctx, host_storage(data, self.dtype)
                                       if data.dtype == np.float32 else data)

    def layout(self, shape: GroupedAttentionShape) -> PackedLayout:
        return packed_layout(shape.q_tensor_len(), shape.lse_len(), self.dtype)

    def forward_resident(self, q, k, v, shape: GroupedAttentionShape,
                         config: FlatAttentionConfig,
                         rotary: Optional[RotaryEmbeddingConfig],
                         out: Optional[DeviceBuffer] = None) -> DeviceBuffer:
        lay = self.layout(shape)
        out = out or DeviceBuffer(self.ctx, lay.combined_bytes)
        rot = ctypes.byref(rotary.c()) if rotary is not None else None
        check(lib().fa_forward_gqa_rope(self.ctx.handle, q.ptr, q.nbytes, k.ptr, v.ptr,
                                        min(k.nbytes, v.nbytes), out.ptr, out.nbytes,
                                        ctypes.byref(shape.c()), ctypes.byref(config.c()), rot,
                                        self.dtype))
        return out

    def prepare(self, q, k, v, out, shape: GroupedAttentionShape, config: FlatAttentionConfig,
                rotary: Optional[RotaryEmbeddingConfig]) -> "PreparedGroupedForward":
        """PreparedGroupedForward::prepare src/wgpu_forward_grouped.rs:352: bind the buffers,
        resolve the variant, own the RoPE table and workspaces; launches only enqueue."""
        h = ctypes.c_void_p()
        rot = ctypes.byref(rotary.c()) if rotary is not None else None
        check(lib().fa_prepare_gqa_rope(self.ctx.handle, q.ptr, q.nbytes, k.ptr, v.ptr,
                                        min(k.nbytes, v.nbytes), out.ptr, out.nbytes,
                                        ctypes.byref(shape.c()), ctypes.byref(config.c()), rot,
                                        self.dtype, ctypes.byref(h)))
        return PreparedGroupedForward(self.ctx, h.value, (q, k, v, out))

    def encode_prepared(self, prepared: "PreparedGroupedForward"):
        """encode_prepared src/wgpu_forward_grouped.rs:496."""
        check(lib().fa_launch_prepared(self.ctx.handle, prepared.handle))
        return prepared.layout()

    def download_attention(self, out: DeviceBuffer, shape) -> FlatAttentionOutput:
        return download_attention(out, self.layout(shape), self.dtype)

    def forward(self, q, k, v, shape: GroupedAttentionShape, config: FlatAttentionConfig,
                rotary: Optional[RotaryEmbeddingConfig]) -> FlatAttentionOutput:
        qs, ks, vs = (host_storage(x, self.dtype) for x in (q, k, v))
        out = np.empty(shape.q_tensor_len(), storage_np_dtype(self.dtype))
        lse = np.empty(shape.lse_len(), np.float32)
        rot = ctypes.byref(rotary.c()) if rotary is not None else None
        check(lib().fa_forward_gqa_rope_host(self.ctx.handle, qs.ctypes.data, ks.ctypes.data,
                                             vs.ctypes.data, qs.size, ks.size, vs.size,
                                             ctypes.byref(shape.c()), ctypes.byref(config.c()),
                                             rot, self.dtype, out.ctypes.data, lse.ctypes.data))
        return FlatAttentionOutput(out, lse)

    def runtime_telemetry(self, shape: Optional[GroupedAttentionShape] = None,
                          config: Optional[FlatAttentionConfig] = None,
                          rotary: Optional[RotaryEmbeddingConfig] = None) -> RuntimeDispatchTelemetry:
        """Passive snapshot for `shape` (no device work), else the last dispatch's record."""
        if shape is None:
            return self.ctx.last_telemetry()
        return self.ctx.forward_telemetry(shape, config, rotary, self.dtype)


class PreparedGroupedForward:
    """PreparedGroupedForward src/wgpu_forward_grouped.rs:352-513 (owns its device state)."""

    def __init__(self, ctx: HipContext, handle: int, buffers):
        self.ctx, self.handle = ctx, handle
        self._buffers = buffers  # the bound buffers stay alive with the prepared forward
        ctx._adopt(self)  # released before its context is destroyed

    def layout(self) -> PackedLayout:
        lay = L.PackedLayoutC()
        check(lib().fa_prepared_forward_layout(self.handle, ctypes.byref(lay)))
        return PackedLayout(lay.output_elements, lay.lse_elements, lay.output_bytes,
                            lay.lse_byte_offset, lay.combined_bytes)

    def release(self):
        if self.handle:
            lib().fa_prepared_forward_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class HipAsymmetricProjectionPipeline:
    """ExternalAsymmetricProjectionRotaryGroupedPipeline src/wgpu_external_asymmetric.rs
    (rectangular projection-layout GQA + RoPE; encode :192 / encode_pre_rotated_k :203).

    ``decode_kv_reuse=True`` (with_decode_kv_reuse :81) enables the opt-in M48 q_len = 1
    candidate, encode_pre_rotated_k_decode_kv_reuse; encode and encode_pre_rotated_k keep their
    route either way."""

    def __init__(self, ctx: HipContext, dtype: int = L.DTYPE_F32, decode_kv_reuse: bool = False):
        self.ctx = ctx
        self.dtype = dtype
        self.decode_kv_reuse = bool(decode_kv_reuse)

    @classmethod
    def with_decode_kv_reuse(cls, ctx: HipContext, enable_candidate: bool,
                             dtype: int = L.DTYPE_F32) -> "HipAsymmetricProjectionPipeline":
        return cls(ctx, dtype, decode_kv_reuse=enable_candidate)

    def create_output_buffer(self, shape: AsymmetricGroupedAttentionShape) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, self.layout(shape).combined_bytes)

    def layout(self, shape: AsymmetricGroupedAttentionShape) -> PackedLayout:
        return packed_layout(shape.q_tensor_len(), shape.lse_len(), self.dtype)

    def encode(self, q, k, v, out, shape, config, rotary=None, rotate_k=True):
        rot = ctypes.byref(rotary.c()) if rotary is not None else None
        check(lib().fa_forward_projection_asymmetric(
            self.ctx.handle, q.ptr, q.nbytes, k.ptr, v.ptr, min(k.nbytes, v.nbytes), out.ptr,
            out.nbytes, ctypes.byref(shape.c()), ctypes.byref(config.c()), rot, int(rotate_k),
            self.dtype))

    def encode_pre_rotated_k(self, q, k, v, out, shape, config, rotary):
        self.encode(q, k, v, out, shape, config, rotary, rotate_k=False)

    def encode_pre_rotated_k_decode_kv_reuse(self, q, k, v, out, shape, config,
                                             rotary) -> PackedLayout:
        """encode_pre_rotated_k_decode_kv_reuse :216 (M48): q_len = 1 decode over pre-rotated K
        whose K/V tiles are read once per GQA group; CandidateNotEnabled unless the pipeline was
        built with the candidate."""
        if not self.decode_kv_reuse:
            raise L.FlatHipError(34, "external FLAT candidate M48 was not enabled")
        check(lib().fa_forward_projection_asymmetric_decode_kv_reuse(
            self.ctx.handle, q.ptr, q.nbytes, k.ptr, v.ptr, min(k.nbytes, v.nbytes), out.ptr,
            out.nbytes, ctypes.byref(shape.c()), ctypes.byref(config.c()),
            ctypes.byref(rotary.c()), self.dtype))
        return self.layout(shape)


class HipProjectionRotaryGroupedPipeline:
    """ExternalProjectionRotaryGroupedPipeline src/wgpu_external.rs:124 (equal-length GQA + RoPE
    in projection layout [batch, seq, heads*head_dim]; Q and K rotated from
    rotary.position_offset, causal within the sequence). encode :206 is the asymmetric pass with
    query_len = kv_len, causal offset 0 and both RoPE offsets at rotary.position_offset."""

    def __init__(self, ctx: HipContext, dtype: int = L.DTYPE_F32):
        self.ctx = ctx
        self.dtype = dtype

    def layout(self, shape: GroupedAttentionShape) -> PackedLayout:  # :159
        return packed_layout(shape.q_tensor_len(), shape.lse_len(), self.dtype)

    def create_output_buffer(self, shape: GroupedAttentionShape) -> DeviceBuffer:  # :184
        return DeviceBuffer(self.ctx, self.layout(shape).combined_bytes)

    def encode(self, q, k, v, out, shape: GroupedAttentionShape, config: FlatAttentionConfig,
               rotary: RotaryEmbeddingConfig) -> PackedLayout:
        ash = AsymmetricGroupedAttentionShape(shape.batch, shape.q_heads, shape.kv_heads,
                                              shape.seq_len, shape.seq_len, shape.head_dim, 0)
        rot = AsymmetricRotaryEmbeddingConfig(rotary.theta, rotary.position_offset,
                                              rotary.position_offset)
        check(lib().fa_forward_projection_asymmetric(
            self.ctx.handle, q.ptr, q.nbytes, k.ptr, v.ptr, min(k.nbytes, v.nbytes), out.ptr,
            out.nbytes, ctypes.byref(ash.c()), ctypes.byref(config.c()), ctypes.byref(rot.c()),
            1, self.dtype))
        return self.layout(shape)


@dataclass(frozen=True)
class VariableLengthSequenceMetadata:
    """VariableLengthSequenceMetadata src/wgpu_external_variable.rs:25."""
    active_query_len: int
    active_kv_len: int
    query_position_offset: int
    query_rope_position_offset: int


@dataclass(frozen=True)
class VariableLengthRotaryEmbeddingConfig:
    """VariableLengthRotaryEmbeddingConfig src/wgpu_external_variable.rs:40."""
    theta: float
    kv_position_offset: int = 0


class HipVariableProjectionPipeline:
    """ExternalVariableProjectionRotaryGroupedPipeline src/wgpu_external_variable.rs:66 (M12:
    padded variable-length projection-layout GQA + RoPE; padded query rows O = 0, LSE = -inf)."""

    def __init__(self, ctx: HipContext, dtype: int = L.DTYPE_F32):
        self.ctx = ctx
        self.dtype = dtype

    def layout(self, shape: AsymmetricGroupedAttentionShape) -> PackedLayout:
        return packed_layout(shape.q_tensor_len(), shape.lse_len(), self.dtype)

    def create_output_buffer(self, shape: AsymmetricGroupedAttentionShape) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, self.layout(shape).combined_bytes)

    def encode(self, q, k, v, out_and_lse, shape: AsymmetricGroupedAttentionShape,
               metadata, config: FlatAttentionConfig,
               rotary: VariableLengthRotaryEmbeddingConfig) -> PackedLayout:
        arr = (L.VariableSequenceC * max(len(metadata), 1))(
            *[L.VariableSequenceC(m.active_query_len, m.active_kv_len, m.query_position_offset,
                                  m.query_rope_position_offset) for m in metadata])
        check(lib().fa_forward_projection_variable(
            self.ctx.handle, q.ptr, q.nbytes, k.ptr, v.ptr, min(k.nbytes, v.nbytes),
            out_and_lse.ptr, out_and_lse.nbytes, ctypes.byref(shape.c()), arr, len(metadata),
            ctypes.byref(config.c()), rotary.theta, rotary.kv_position_offset, self.dtype))
        return self.layout(shape)


class HipChunkedProjectionPrefillPipeline:
    """WgpuChunkedProjectionPrefillPipeline src/wgpu_chunked_prefill.rs:99."""

    def __init__(self, ctx: HipContext, dtype: int = L.DTYPE_F32):
        self.ctx = ctx
        self.dtype = dtype

    def layout(self, shape: GroupedAttentionShape) -> PackedLayout:
        return packed_layout(shape.q_tensor_len(), shape.lse_len(), self.dtype)

    def create_output_buffer(self, shape: GroupedAttentionShape) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, self.layout(shape).combined_bytes)

    def encode(self, q, k, v, out_and_lse, shape: GroupedAttentionShape,
               config: FlatAttentionConfig, rotary: RotaryEmbeddingConfig,
               query_chunk_size: int):
        check(lib().fa_chunked_prefill(self.ctx.handle, q.ptr, q.nbytes, k.ptr, v.ptr,
                                       min(k.nbytes, v.nbytes), out_and_lse.ptr,
                                       out_and_lse.nbytes, ctypes.byref(shape.c()),
                                       ctypes.byref(config.c()), ctypes.byref(rotary.c()),
                                       query_chunk_size, self.dtype))


# ----------------------------------------------------------------------------- paged KV

@dataclass(frozen=True)
class PagedKvConfig:
    """PagedKvConfig src/paged_kv.rs:4."""
    page_size: int
    physical_pages: int


@dataclass(frozen=True)
class PagedKvAddress:
    physical_page: int
    offset_in_page: int
    generation: int


@dataclass(frozen=True)
class PagedKvTelemetry:
    live_tokens: int
    capacity_tokens: int
    mapped_pages: int
    free_pages: int
    internal_fragmentation_tokens: int
    generation: int


class PagedKvTable:
    """PagedKvTable src/paged_kv.rs:76 (host metadata, lowest free page first)."""

    def __init__(self, config: PagedKvConfig, _handle=None, _owned=True):
        if _handle is None:
            h = L.VP()
            check(lib().fa_kv_table_create(config.page_size, config.physical_pages,
                                           ctypes.byref(h)))
            _handle = h.value
        self.config = config
        self.handle = _handle
        self._owned = _owned

    def __del__(self):
        if getattr(self, "_owned", False) and self.handle:
            lib().fa_kv_table_destroy(self.handle)
            self.handle = None

    def clone(self) -> "PagedKvTable":
        h = L.VP()
        check(lib().fa_kv_table_clone(self.handle, ctypes.byref(h)))
        return PagedKvTable(self.config, h.value, True)

    def __len__(self):
        return int(lib().fa_kv_table_len(self.handle))

    def append(self, tokens: int):
        check(lib().fa_kv_table_append(self.handle, tokens))

    def address(self, logical_token: int) -> Optional[PagedKvAddress]:
        a = L.KvAddressC()
        rc = lib().fa_kv_table_address(self.handle, logical_token, ctypes.byref(a))
        if rc == 25:  # unmapped -> None (Option::None in the reference)
            return None
        check(rc)
        return PagedKvAddress(a.physical_page, a.offset_in_page, a.generation)

    def telemetry(self) -> PagedKvTelemetry:
        t = L.KvTelemetryC()
        check(lib().fa_kv_table_telemetry(self.handle, ctypes.byref(t)))
        return PagedKvTelemetry(t.live_tokens, t.capacity_tokens, t.mapped_pages, t.free_pages,
                                t.internal_fragmentation_tokens, t.generation)

    def reset(self):
        check(lib().fa_kv_table_reset(self.handle))

    def block_row(self) -> np.ndarray:
        """WgpuPagedKvTable::from_table src/wgpu_paged_decode.rs:162."""
        n = L.U64()
        check(lib().fa_kv_table_block_row(self.handle, None, 0, ctypes.byref(n)))
        row = np.empty(n.value, np.int32)
        check(lib().fa_kv_table_block_row(self.handle, row.ctypes.data, n.value, ctypes.byref(n)))
        return row


class HipPagedKvCache:
    """WgpuPagedKvCache src/wgpu_paged_kv_cache.rs:76: [pages, page_size, kv_heads*head_dim]."""

    def __init__(self, ctx: HipContext, config: PagedKvConfig, kv_heads: int, head_dim: int,
                 dtype: int = L.DTYPE_F32):
        h = L.VP()
        check(lib().fa_paged_cache_create(ctx.handle, config.page_size, config.physical_pages,
                                          kv_heads, head_dim, dtype, ctypes.byref(h)))
        self.ctx = ctx
        self.handle = h.value
        self.config = config
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        ctx._adopt(self)

    def release(self):
        if getattr(self, "handle", None) and self.ctx.handle:
            lib().fa_paged_cache_destroy(self.handle)
        self.handle = None

    def __del__(self):
        self.release()

    def table(self) -> PagedKvTable:
        return PagedKvTable(self.config, lib().fa_paged_cache_table(self.handle), False)

    def k_buffer(self) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, lib().fa_paged_cache_bytes(self.handle),
                            lib().fa_paged_cache_k(self.handle), owned=False)

    def v_buffer(self) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, lib().fa_paged_cache_bytes(self.handle),
                            lib().fa_paged_cache_v(self.handle), owned=False)

    def record_append(self, k_source: DeviceBuffer, v_source: DeviceBuffer, append_len: int,
                      rotate_k: Optional[RotaryEmbeddingConfig] = None) -> int:
        n = L.U64()
        rot = ctypes.byref(rotate_k.c()) if rotate_k is not None else None
        check(lib().fa_paged_cache_append(self.handle, k_source.ptr, v_source.ptr,
                                          min(k_source.nbytes, v_source.nbytes), append_len, rot,
                                          ctypes.byref(n)))
        return n.value

    def reset(self):
        check(lib().fa_paged_cache_reset(self.handle))


class PagedDecodePlan:
    """Prepared batched paged decode (validated, resident block tables + split schedule)."""

    def __init__(self, ctx: HipContext, block_tables: np.ndarray, ctx_lens: np.ndarray,
                 page_size: int, physical_pages: int, q_heads: int, kv_heads: int,
                 head_dim: int, config: FlatAttentionConfig, theta: float, dtype: int,
                 q_positions: Optional[np.ndarray] = None):
        bt = np.ascontiguousarray(block_tables, np.int32)
        cl = np.ascontiguousarray(ctx_lens, np.int32)
        qp = None if q_positions is None else np.ascontiguousarray(q_positions, np.int32)
        h = L.VP()
        check(lib().fa_paged_decode_prepare(
            ctx.handle, bt.ctypes.data, bt.shape[1], cl.ctypes.data,
            None if qp is None else qp.ctypes.data, cl.shape[0], page_size, physical_pages,
            q_heads, kv_heads, head_dim, ctypes.byref(config.c()), theta, dtype,
            ctypes.byref(h)))
        self.ctx, self.handle, self.dtype = ctx, h.value, dtype
        self.n_seqs, self.q_heads, self.head_dim = cl.shape[0], q_heads, head_dim
        ctx._adopt(self)

    def release(self):
        if getattr(self, "handle", None) and self.ctx.handle:
            lib().fa_paged_decode_plan_destroy(self.handle)
        self.handle = None

    def __del__(self):
        self.release()

    def layout(self) -> PackedLayout:
        n = self.n_seqs * self.q_heads
        return packed_layout(n * self.head_dim, n, self.dtype)

    def info(self):
        a, b, c = L.U64(), L.U64(), L.U64()
        check(lib().fa_paged_decode_plan_info(self.handle, ctypes.byref(a), ctypes.byref(b),
                                              ctypes.byref(c)))
        return {"split_tokens": a.value, "work_items": b.value, "workspace_bytes": c.value}

    def set_split(self, split_tokens: int):
        check(lib().fa_paged_decode_plan_set_split(self.ctx.handle, self.handle, split_tokens))

    def launch(self, q: DeviceBuffer, k_pool: DeviceBuffer, v_pool: DeviceBuffer,
               out_and_lse: DeviceBuffer):
        check(lib().fa_paged_decode_launch(self.ctx.handle, self.handle, q.ptr, q.nbytes,
                                           k_pool.ptr, v_pool.ptr,
                                           min(k_pool.nbytes, v_pool.nbytes), out_and_lse.ptr,
                                           out_and_lse.nbytes))


def paged_decode_noalloc(ctx: HipContext, block_tables: np.ndarray, ctx_lens: np.ndarray,
                         page_size: int, physical_pages: int, q_heads: int, kv_heads: int,
                         head_dim: int, config: FlatAttentionConfig, theta: float, dtype: int,
                         q: DeviceBuffer, k_pool: DeviceBuffer, v_pool: DeviceBuffer,
                         out_and_lse: DeviceBuffer,
                         q_positions: Optional[np.ndarray] = None) -> PackedLayout:
    """Allocation-free batched paged decode (no reference counterpart): PagedDecodePlan's
    prepare + launch in one call whose device state lives in the library's static per-device
    scratch. Calls from different contexts on one GPU are ordered on the GPU (each waits for the
    previous user's kernels); refused while the context's stream is being captured."""
    bt = np.ascontiguousarray(block_tables, np.int32)
    cl = np.ascontiguousarray(ctx_lens, np.int32)
    qp = None if q_positions is None else np.ascontiguousarray(q_positions, np.int32)
    check(lib().fa_paged_decode_noalloc(
        ctx.handle, bt.ctypes.data, bt.shape[1], cl.ctypes.data,
        None if qp is None else qp.ctypes.data, cl.shape[0], page_size, physical_pages, q_heads,
        kv_heads, head_dim, ctypes.byref(config.c()), theta, dtype, q.ptr, q.nbytes, k_pool.ptr,
        v_pool.ptr, min(k_pool.nbytes, v_pool.nbytes), out_and_lse.ptr, out_and_lse.nbytes))
    n = cl.shape[0] * q_heads
    return packed_layout(n * head_dim, n, dtype)


class HipPagedDecodePipeline:
    """WgpuPagedDecodePipeline src/wgpu_paged_decode.rs:244 (single sequence over a cache)."""

    def __init__(self, ctx: HipContext, dtype: int = L.DTYPE_F32):
        self.ctx = ctx
        self.dtype = dtype

    def layout(self, q_heads: int, head_dim: int) -> PackedLayout:
        return packed_layout(q_heads * head_dim, q_heads, self.dtype)

    def create_output_buffer(self, q_heads: int, head_dim: int) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, self.layout(q_heads, head_dim).combined_bytes)

    def encode(self, q: DeviceBuffer, cache: HipPagedKvCache, out_and_lse: DeviceBuffer,
               q_heads: int, config: FlatAttentionConfig, theta: float,
               q_rope_position: int) -> PackedLayout:
        check(lib().fa_paged_cache_decode(self.ctx.handle, cache.handle, q.ptr, q.nbytes,
                                          q_heads, ctypes.byref(config.c()), theta,
                                          q_rope_position, out_and_lse.ptr, out_and_lse.nbytes))
        return self.layout(q_heads, cache.head_dim)


class HipResidentKvCache:
    """WgpuResidentKvCache src/wgpu_kv_cache.rs:79: fixed-capacity K/V
    [batch, capacity, kv_heads*head_dim], one live length shared by the batch."""

    def __init__(self, ctx: HipContext, batch: int, kv_heads: int, capacity: int, head_dim: int,
                 dtype: int = L.DTYPE_F32):
        h = L.VP()
        check(lib().fa_resident_cache_create(ctx.handle, batch, kv_heads, capacity, head_dim,
                                             dtype, ctypes.byref(h)))
        self.ctx, self.handle, self.dtype = ctx, h.value, dtype
        self.batch, self.kv_heads, self.capacity, self.head_dim = batch, kv_heads, capacity, head_dim
        ctx._adopt(self)

    def release(self):
        if getattr(self, "handle", None) and self.ctx.handle:
            lib().fa_resident_cache_destroy(self.handle)
        self.handle = None

    def __del__(self):
        self.release()

    def __len__(self) -> int:
        return lib().fa_resident_cache_len(self.handle)

    def is_empty(self) -> bool:
        return len(self) == 0

    def remaining_capacity(self) -> int:  # :184
        return self.capacity - len(self)

    def k_buffer(self) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, lib().fa_resident_cache_bytes(self.handle),
                            lib().fa_resident_cache_k(self.handle), owned=False)

    def v_buffer(self) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, lib().fa_resident_cache_bytes(self.handle),
                            lib().fa_resident_cache_v(self.handle), owned=False)

    def record_append(self, k_source: DeviceBuffer, v_source: DeviceBuffer, append_len: int) -> int:
        """record_append :212 (sources [batch, append_len, kv_heads*head_dim], K pre-rotated)."""
        n = L.U64()
        check(lib().fa_resident_cache_append(self.handle, k_source.ptr, v_source.ptr,
                                             min(k_source.nbytes, v_source.nbytes), append_len,
                                             ctypes.byref(n)))
        return n.value

    def reset(self):
        check(lib().fa_resident_cache_reset(self.handle))


class ResidentDecodePlan(PagedDecodePlan):
    """WgpuResidentDecodePipeline::encode_external_pre_rotated_k src/wgpu_decode.rs:301 over
    framework-owned [batch, capacity, kv_heads*head_dim] K (pre-rotated) / V; launch() takes the
    two K/V buffers in place of a page pool."""

    def __init__(self, ctx: HipContext, batch: int, capacity: int, kv_len: int, q_heads: int,
                 kv_heads: int, head_dim: int, config: FlatAttentionConfig, theta: float,
                 q_rope_position: int, dtype: int):
        h = L.VP()
        check(lib().fa_resident_decode_prepare(ctx.handle, batch, capacity, kv_len, q_heads,
                                               kv_heads, head_dim, ctypes.byref(config.c()),
                                               theta, q_rope_position, dtype, ctypes.byref(h)))
        self.ctx, self.handle, self.dtype = ctx, h.value, dtype
        self.n_seqs, self.q_heads, self.head_dim = batch, q_heads, head_dim
        ctx._adopt(self)


class HipResidentDecodePipeline:
    """WgpuResidentDecodePipeline src/wgpu_decode.rs:214 (q_len = 1 decode over resident K/V)."""

    def __init__(self, ctx: HipContext, dtype: int = L.DTYPE_F32):
        self.ctx = ctx
        self.dtype = dtype

    def layout(self, batch: int, q_heads: int, head_dim: int) -> PackedLayout:
        return packed_layout(batch * q_heads * head_dim, batch * q_heads, self.dtype)

    def create_output_buffer(self, cache: HipResidentKvCache, q_heads: int) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, self.layout(cache.batch, q_heads, cache.head_dim).combined_bytes)

    def encode(self, q: DeviceBuffer, cache: HipResidentKvCache, out_and_lse: DeviceBuffer,
               q_heads: int, config: FlatAttentionConfig, theta: float,
               q_rope_position: int) -> PackedLayout:
        """encode :265 (ResidentDecodePass over FLAT's cache)."""
        check(lib().fa_resident_cache_decode(self.ctx.handle, cache.handle, q.ptr, q.nbytes,
                                             q_heads, ctypes.byref(config.c()), theta,
                                             q_rope_position, out_and_lse.ptr, out_and_lse.nbytes))
        return self.layout(cache.batch, q_heads, cache.head_dim)

    def encode_external_pre_rotated_k(self, q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer,
                                      out_and_lse: DeviceBuffer,
                                      shape: "AsymmetricGroupedAttentionShape",
                                      config: FlatAttentionConfig,
                                      rotary: "AsymmetricRotaryEmbeddingConfig",
                                      kv_capacity: int) -> PackedLayout:
        """encode_external_pre_rotated_k :301. shape.query_len must be 1 (else InvalidQueryLen
        in the reference; here LengthMismatch)."""
        if shape.query_len != 1:
            raise L.FlatHipError(7, f"specialized resident decode requires query_len=1, got "
                                  f"{shape.query_len}")
        # validate_external_semantics :419: causal visibility uses the shape's query position
        # (RoPE uses the rotary one); a q_len = 1 decode then attends every live row either way
        if config.causal and shape.query_position_offset + 1 < shape.kv_len:
            raise L.FlatHipError(27, f"resident causal decode query position "
                                   f"{shape.query_position_offset} cannot see all {shape.kv_len} "
                                   f"live KV rows")
        plan = ResidentDecodePlan(self.ctx, shape.batch, kv_capacity, shape.kv_len, shape.q_heads,
                                  shape.kv_heads, shape.head_dim,
                                  FlatAttentionConfig(False, config.softmax_scale), rotary.theta,
                                  rotary.query_position_offset, self.dtype)
        plan.launch(q, k, v, out_and_lse)
        layout = plan.layout()
        plan.release()
        return layout


class PagedChunkedPrefillPlan:
    """Chunked prefill of a query chunk over a shared paged cache (pre-rotated K)."""

    def __init__(self, ctx: HipContext, block_tables: np.ndarray, page_size: int,
                 physical_pages: int, shape: AsymmetricGroupedAttentionShape,
                 config: FlatAttentionConfig, rotary: AsymmetricRotaryEmbeddingConfig,
                 dtype: int):
        bt = np.ascontiguousarray(block_tables, np.int32)
        h = L.VP()
        check(lib().fa_chunked_prefill_paged_prepare(
            ctx.handle, bt.ctypes.data, bt.shape[1], page_size, physical_pages,
            ctypes.byref(shape.c()), ctypes.byref(config.c()), ctypes.byref(rotary.c()), dtype,
            ctypes.byref(h)))
        self.ctx, self.handle, self.dtype, self.shape = ctx, h.value, dtype, shape
        ctx._adopt(self)

    def release(self):
        if getattr(self, "handle", None) and self.ctx.handle:
            lib().fa_prefill_plan_destroy(self.handle)
        self.handle = None

    def __del__(self):
        self.release()

    def layout(self) -> PackedLayout:
        return packed_layout(self.shape.q_tensor_len(), self.shape.lse_len(), self.dtype)

    def launch(self, q, k_pool, v_pool, out_and_lse):
        check(lib().fa_chunked_prefill_paged_launch(self.ctx.handle, self.handle, q.ptr,
                                                    q.nbytes, k_pool.ptr, v_pool.ptr,
                                                    min(k_pool.nbytes, v_pool.nbytes),
                                                    out_and_lse.ptr, out_and_lse.nbytes))


def paged_append_batched(ctx: HipContext, block_tables: np.ndarray, start_lens: np.ndarray,
                         append_len: int, page_size: int, physical_pages: int, kv_heads: int,
                         head_dim: int, k_src: DeviceBuffer, v_src: DeviceBuffer,
                         k_pool: DeviceBuffer, v_pool: DeviceBuffer,
                         rotary: Optional[RotaryEmbeddingConfig], dtype: int):
    """Batched record_append with RoPE-on-append."""
    bt = np.ascontiguousarray(block_tables, np.int32)
    st = np.ascontiguousarray(start_lens, np.int32)
    rot = ctypes.byref(rotary.c()) if rotary is not None else None
    check(lib().fa_paged_append_batched(ctx.handle, bt.ctypes.data, bt.shape[1], st.ctypes.data,
                                        st.shape[0], append_len, page_size, physical_pages,
                                        kv_heads, head_dim, k_src.ptr, v_src.ptr,
                                        min(k_src.nbytes, v_src.nbytes), k_pool.ptr, v_pool.ptr,
                                        min(k_pool.nbytes, v_pool.nbytes), rot, dtype))


# ----------------------------------------------------------------------------- backward

@dataclass
class FlatAttentionBackwardOutput:
    """FlatAttentionBackwardOutput src/backward.rs:12 (dq, dk, dv as float32 arrays)."""
    dq: np.ndarray
    dk: np.ndarray
    dv: np.ndarray


@dataclass(frozen=True)
class GroupedBackwardRecomputeLayout:
    """GroupedBackwardRecomputeLayout src/wgpu_backward_grouped.rs:18. Offsets and sizes are in
    bytes: tensors are stored in the pipeline dtype and LSE in f32 (for f32 every offset is the
    reference's element offset times 4)."""
    q_elements: int
    kv_elements: int
    lse_elements: int
    packed_forward_bytes: int
    gradient_bytes: int
    q_offset: int
    k_offset: int
    v_offset: int
    d_out_offset: int
    output_offset: int
    lse_offset: int
    dq_offset: int
    dk_offset: int
    dv_offset: int


@dataclass(frozen=True)
class PreparedGroupedBackwardRecompute:
    """PreparedGroupedBackwardRecompute src/wgpu_backward_grouped.rs:124: a validated
    (buffers, shape, config) tuple that encode_prepared launches without re-deriving it."""
    packed_forward: DeviceBuffer
    packed_grads: DeviceBuffer
    shape: GroupedAttentionShape
    config: FlatAttentionConfig
    layout: GroupedBackwardRecomputeLayout
    scale: float


def grouped_backward_layout(shape: GroupedAttentionShape,
                            dtype: int) -> GroupedBackwardRecomputeLayout:
    """WgpuGroupedBackwardRecomputePipeline::layout src/wgpu_backward_grouped.rs:181."""
    c = L.BackwardLayoutC()
    check(lib().fa_backward_grouped_layout(ctypes.byref(shape.c()), dtype, ctypes.byref(c)))
    return GroupedBackwardRecomputeLayout(*(getattr(c, n) for n, _ in c._fields_))


class HipGroupedBackwardRecomputePipeline:
    """WgpuGroupedBackwardRecomputePipeline src/wgpu_backward_grouped.rs:146: recompute
    backward of native GQA/MQA attention over the packed Q|K|V|dO|O|LSE -> dQ|dK|dV contract."""

    def __init__(self, ctx: HipContext, dtype: int = L.DTYPE_F32):
        self.ctx = ctx
        self.dtype = dtype

    def layout(self, shape: GroupedAttentionShape) -> GroupedBackwardRecomputeLayout:
        return grouped_backward_layout(shape, self.dtype)

    def create_gradient_buffer(self, shape: GroupedAttentionShape) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, self.layout(shape).gradient_bytes)

    def prepare(self, packed_forward: DeviceBuffer, packed_grads: DeviceBuffer,
                shape: GroupedAttentionShape,
                config: FlatAttentionConfig) -> PreparedGroupedBackwardRecompute:
        lay = self.layout(shape)
        for name, buf, need in (("Q|K|V|dO|O|LSE", packed_forward, lay.packed_forward_bytes),
                                ("dQ|dK|dV", packed_grads, lay.gradient_bytes)):
            if buf.nbytes < need:
                raise L.FlatHipError(24, f"buffer {name} contains {buf.nbytes} bytes, requires "
                                         f"at least {need}")
        scale = ctypes.c_float()
        check(lib().fa_resolved_scale(ctypes.byref(config.c()), shape.head_dim,
                                      ctypes.byref(scale)))
        return PreparedGroupedBackwardRecompute(packed_forward, packed_grads, shape, config, lay,
                                                scale.value)

    def encode_prepared(self, prepared: PreparedGroupedBackwardRecompute
                        ) -> GroupedBackwardRecomputeLayout:
        p = prepared
        check(lib().fa_backward_grouped_recompute(
            self.ctx.handle, p.packed_forward.ptr, p.packed_forward.nbytes, p.packed_grads.ptr,
            p.packed_grads.nbytes, ctypes.byref(p.shape.c()), ctypes.byref(p.config.c()),
            self.dtype))
        return p.layout

    def encode(self, packed_forward: DeviceBuffer, packed_grads: DeviceBuffer,
               shape: GroupedAttentionShape,
               config: FlatAttentionConfig) -> GroupedBackwardRecomputeLayout:
        return self.encode_prepared(self.prepare(packed_forward, packed_grads, shape, config))

    def encode_tensors(self, q, k, v, d_out, out, lse_ptr: int, dq, dk, dv,
                       shape: GroupedAttentionShape, config: FlatAttentionConfig):
        """fa_backward_grouped over separate device tensors (DeviceBuffer-like objects with
        ``ptr``); ``lse_ptr`` is a raw device address of the f32 LSE rows."""
        check(lib().fa_backward_grouped(self.ctx.handle, q.ptr, k.ptr, v.ptr, d_out.ptr, out.ptr,
                                        lse_ptr, dq.ptr, dk.ptr, dv.ptr,
                                        ctypes.byref(shape.c()), ctypes.byref(config.c()),
                                        self.dtype))

    def download_gradients(self, grads: DeviceBuffer,
                           shape: GroupedAttentionShape) -> FlatAttentionBackwardOutput:
        lay = self.layout(shape)
        sd = storage_np_dtype(self.dtype)
        parts = [grads.download(sd, n, off) for n, off in ((lay.q_elements, lay.dq_offset),
                                                          (lay.kv_elements, lay.dk_offset),
                                                          (lay.kv_elements, lay.dv_offset))]
        return FlatAttentionBackwardOutput(*(storage_to_f32(x, self.dtype) for x in parts))

    def backward(self, q, k, v, d_out, forward: FlatAttentionOutput,
                 shape: GroupedAttentionShape,
                 config: FlatAttentionConfig) -> FlatAttentionBackwardOutput:
        """Host convenience: pack, upload, encode, download (float32 gradients)."""
        packed = pack_grouped_backward_recompute_inputs(q, k, v, d_out, forward, shape,
                                                        self.dtype, self.layout(shape))
        fwd = DeviceBuffer.from_array(self.ctx, packed)
        grads = self.create_gradient_buffer(shape)
        self.encode(fwd, grads, shape, config)
        res = self.download_gradients(grads, shape)
        fwd.free()
        grads.free()
        return res


def pack_grouped_backward_recompute_inputs(q, k, v, d_out, forward: FlatAttentionOutput,
                                           shape: GroupedAttentionShape,
                                           dtype: int = L.DTYPE_F32,
                                           layout: Optional[GroupedBackwardRecomputeLayout] = None
                                           ) -> np.ndarray:
    """pack_grouped_backward_recompute_inputs src/wgpu_backward_grouped.rs:331 as bytes: Q, K,
    V, dO, O in the storage dtype (float32 inputs are converted; storage arrays pass through),
    then LSE f32. Lengths are validated like validate_input (LengthMismatch)."""
    lay = layout or grouped_backward_layout(shape, dtype)
    sd = storage_np_dtype(dtype)
    parts = []
    for name, x, n in (("Q", q, lay.q_elements), ("K", k, lay.kv_elements),
                       ("V", v, lay.kv_elements), ("dO", d_out, lay.q_elements),
                       ("O", forward.output, lay.q_elements)):
        x = np.asarray(x).ravel()
        if x.size != n:
            raise L.FlatHipError(7, f"{name} has {x.size} values, expected {n}")
        parts.append(np.ascontiguousarray(x if x.dtype == sd else host_storage(x, dtype)))
    lse = np.ascontiguousarray(np.asarray(forward.lse, np.float32).ravel())
    if lse.size != lay.lse_elements:
        raise L.FlatHipError(7, f"LSE has {lse.size} values, expected {lay.lse_elements}")
    parts.append(lse)
    return np.concatenate([p.view(np.uint8) for p in parts])


class HipBackwardRecomputePipeline:
    """WgpuBackwardRecomputePipeline src/wgpu_backward.rs:127 (M18 canonical MHA recompute
    backward): the grouped backward with kv_heads == heads over the same packed contract."""

    def __init__(self, ctx: HipContext, dtype: int = L.DTYPE_F32):
        self.ctx = ctx
        self.dtype = dtype

    def layout(self, shape: AttentionShape) -> GroupedBackwardRecomputeLayout:
        c = L.BackwardLayoutC()
        check(lib().fa_backward_layout_mha(ctypes.byref(shape.c()), self.dtype, ctypes.byref(c)))
        return GroupedBackwardRecomputeLayout(*(getattr(c, n) for n, _ in c._fields_))

    def create_gradient_buffer(self, shape: AttentionShape) -> DeviceBuffer:
        return DeviceBuffer(self.ctx, self.layout(shape).gradient_bytes)

    def encode(self, packed_forward: DeviceBuffer, packed_grads: DeviceBuffer,
               shape: AttentionShape, config: FlatAttentionConfig
               ) -> GroupedBackwardRecomputeLayout:
        check(lib().fa_backward_recompute_mha(
            self.ctx.handle, packed_forward.ptr, packed_forward.nbytes, packed_grads.ptr,
            packed_grads.nbytes, ctypes.byref(shape.c()), ctypes.byref(config.c()), self.dtype))
        return self.layout(shape)


def pack_backward_recompute_inputs(q, k, v, d_out, forward: FlatAttentionOutput,
                                   shape: AttentionShape, dtype: int = L.DTYPE_F32) -> np.ndarray:
    """pack_backward_recompute_inputs src/wgpu_backward.rs:282 (bytes, as the grouped packer)."""
    g = GroupedAttentionShape(shape.batch, shape.heads, shape.heads, shape.seq_len,
                              shape.head_dim)
    return pack_grouped_backward_recompute_inputs(q, k, v, d_out, forward, g, dtype)
