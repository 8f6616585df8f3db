"""ctypes binding of ``libflat_hip.so`` (declarations in ``include/flat_hip.h``).

Loading fails loudly when the library has not been built; there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libflat_hip.so")

U64 = ctypes.c_uint64
I32 = ctypes.c_int32
INT = ctypes.c_int
F32 = ctypes.c_float
VP = ctypes.c_void_p
SZ = ctypes.c_size_t
P = ctypes.POINTER

# fa_dtype
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
DTYPE_BYTES = {DTYPE_F32: 4, DTYPE_F16: 2, DTYPE_BF16: 2}

STATUS = {
    0: "Ok", 1: "ZeroDimension", 2: "ShapeOverflow", 3: "InvalidHeadGrouping",
    4: "InvalidRotaryHeadDim", 5: "InvalidRotaryTheta", 6: "PositionOverflow",
    7: "LengthMismatch", 8: "InvalidScale", 9: "NonFiniteInput", 20: "Unavailable",
    21: "UnsupportedHeadDim", 22: "IndexSpaceExceeded", 23: "DispatchLimit",
    24: "BufferTooSmall", 25: "EmptyTable", 26: "TooManyMappedPages",
    27: "CausalVisibilityMismatch", 28: "ZeroQueryChunkSize", 29: "UnsupportedDtype",
    30: "InvalidPage", 31: "EmptyCache", 32: "InvalidCacheLength", 33: "ForeignBuffer", 34: "CandidateNotEnabled",
    35: "UnsupportedCandidateShape", 40: "PagedZeroDimension", 41: "CapacityOverflow",
    42: "CapacityExceeded", 43: "GenerationOverflow", 50: "NullArgument", 60: "Hip",
    61: "ScratchExceeded", 62: "GraphCapture",
}

KERNEL_IDS = {
    0: "None", 1: "PrefillMfmaBf16", 2: "PrefillMfmaF16", 3: "PrefillMfmaF32",
    4: "PrefillMfmaBf16PreRotatedK", 5: "PrefillMfmaF16PreRotatedK",
    6: "PrefillMfmaF32PreRotatedK", 10: "DecodePagedSplitK", 11: "DecodeCombine",
    12: "PagedAppend", 13: "RopeTable", 14: "RopeRotate", 15: "DecodePagedMfma", 16: "TransposeV",
    17: "BackwardRecompute",
}


class AttentionShapeC(ctypes.Structure):
    _fields_ = [("batch", U64), ("heads", U64), ("seq_len", U64), ("head_dim", U64)]


class GroupedShapeC(ctypes.Structure):
    _fields_ = [("batch", U64), ("q_heads", U64), ("kv_heads", U64), ("seq_len", U64),
                ("head_dim", U64)]


class AsymmetricShapeC(ctypes.Structure):
    _fields_ = [("batch", U64), ("q_heads", U64), ("kv_heads", U64), ("query_len", U64),
                ("kv_len", U64), ("head_dim", U64), ("query_position_offset", U64)]


class ConfigC(ctypes.Structure):
    _fields_ = [("causal", I32), ("has_softmax_scale", I32), ("softmax_scale", F32)]


class RotaryC(ctypes.Structure):
    _fields_ = [("theta", F32), ("position_offset", U64)]


class VariableSequenceC(ctypes.Structure):
    _fields_ = [("active_query_len", U64), ("active_kv_len", U64),
                ("query_position_offset", U64), ("query_rope_position_offset", U64)]


class AsymmetricRotaryC(ctypes.Structure):
    _fields_ = [("theta", F32), ("query_position_offset", U64), ("kv_position_offset", U64)]


class PackedLayoutC(ctypes.Structure):
    _fields_ = [("output_elements", U64), ("lse_elements", U64), ("output_bytes", U64),
                ("lse_byte_offset", U64), ("combined_bytes", U64)]


class BackwardLayoutC(ctypes.Structure):
    _fields_ = [(n, U64) for n in (
        "q_elements", "kv_elements", "lse_elements", "packed_forward_bytes", "gradient_bytes",
        "q_offset", "k_offset", "v_offset", "d_out_offset", "output_offset", "lse_offset",
        "dq_offset", "dk_offset", "dv_offset")]


class TelemetryC(ctypes.Structure):
    _fields_ = [("kernel_id", I32), ("kernel_name", ctypes.c_char * 64), ("query_rows", ctypes.c_uint32),
                ("kv_rows", ctypes.c_uint32), ("workgroups", ctypes.c_uint32 * 3),
                ("workgroup_size", ctypes.c_uint32), ("dispatch_count", ctypes.c_uint32),
                ("temporary_allocation_count", ctypes.c_uint32),
                ("temporary_allocation_bytes", U64), ("splits", ctypes.c_uint32),
                ("has_fallback_reason", I32), ("fallback_reason", ctypes.c_char * 128),
                ("device_name", ctypes.c_char * 64), ("device_arch", ctypes.c_char * 32),
                ("device_fingerprint", U64)]


class KvAddressC(ctypes.Structure):
    _fields_ = [("physical_page", U64), ("offset_in_page", U64), ("generation", U64)]


class KvTelemetryC(ctypes.Structure):
    _fields_ = [("live_tokens", U64), ("capacity_tokens", U64), ("mapped_pages", U64),
                ("free_pages", U64), ("internal_fragmentation_tokens", U64), ("generation", U64)]


# name -> (restype, argtypes)
PROTOTYPES = {
    "fa_abi_version": (INT, []),
    "fa_status_string": (ctypes.c_char_p, [INT]),
    "fa_last_error_message": (ctypes.c_char_p, []),
    "fa_resolved_scale": (INT, [P(ConfigC), U64, P(F32)]),
    "fa_packed_layout_for": (INT, [U64, U64, INT, P(PackedLayoutC)]),
    "fa_ctx_create": (INT, [INT, P(VP)]),
    "fa_ctx_destroy": (INT, [VP]),
    "fa_ctx_stream": (VP, [VP]),
    "fa_ctx_synchronize": (INT, [VP]),
    "fa_graph_capture_begin": (INT, [VP]),
    "fa_graph_capture_end": (INT, [VP, P(VP)]),
    "fa_graph_launch": (INT, [VP, VP]),
    "fa_graph_destroy": (INT, [VP]),
    "fa_ctx_device_name": (INT, [VP, ctypes.c_char_p, SZ]),
    "fa_ctx_set_prefill_policy": (INT, [VP, I32]),
    "fa_ctx_set_prefill_kernel": (INT, [VP, I32]),
    "fa_kernel_variant_for_shape": (INT, [VP, U64, I32, INT, P(I32)]),
    "fa_buf_alloc": (INT, [VP, SZ, P(VP)]),
    "fa_buf_free": (INT, [VP, VP]),
    "fa_buf_upload": (INT, [VP, VP, VP, SZ]),
    "fa_buf_download": (INT, [VP, VP, VP, SZ]),
    "fa_buf_fill_u32": (INT, [VP, VP, ctypes.c_uint32, SZ]),
    "fa_forward_mha": (INT, [VP, VP, VP, VP, SZ, VP, SZ, P(AttentionShapeC), P(ConfigC), INT]),
    "fa_forward_gqa_rope": (INT, [VP, VP, SZ, VP, VP, SZ, VP, SZ, P(GroupedShapeC), P(ConfigC),
                                  P(RotaryC), INT]),
    "fa_prepare_gqa_rope": (INT, [VP, VP, SZ, VP, VP, SZ, VP, SZ, P(GroupedShapeC), P(ConfigC),
                                  P(RotaryC), INT, P(VP)]),
    "fa_prepare_mha": (INT, [VP, VP, VP, VP, SZ, VP, SZ, P(AttentionShapeC), P(ConfigC), INT,
                             P(VP)]),
    "fa_launch_prepared": (INT, [VP, VP]),
    "fa_prepared_forward_layout": (INT, [VP, P(PackedLayoutC)]),
    "fa_prepared_forward_destroy": (INT, [VP]),
    "fa_forward_mha_host": (INT, [VP, VP, VP, VP, U64, U64, U64, P(AttentionShapeC), P(ConfigC),
                                  INT, VP, VP]),
    "fa_forward_gqa_rope_host": (INT, [VP, VP, VP, VP, U64, U64, U64, P(GroupedShapeC),
                                       P(ConfigC), P(RotaryC), INT, VP, VP]),
    "fa_forward_projection_asymmetric": (INT, [VP, VP, SZ, VP, VP, SZ, VP, SZ,
                                               P(AsymmetricShapeC), P(ConfigC),
                                               P(AsymmetricRotaryC), I32, INT]),
    "fa_forward_projection_asymmetric_decode_kv_reuse": (INT, [
        VP, VP, SZ, VP, VP, SZ, VP, SZ, P(AsymmetricShapeC), P(ConfigC), P(AsymmetricRotaryC),
        INT]),
    "fa_chunked_prefill": (INT, [VP, VP, SZ, VP, VP, SZ, VP, SZ, P(GroupedShapeC), P(ConfigC),
                                 P(RotaryC), U64, INT]),
    "fa_kv_table_create": (INT, [U64, U64, P(VP)]),
    "fa_kv_table_destroy": (INT, [VP]),
    "fa_kv_table_clone": (INT, [VP, P(VP)]),
    "fa_kv_table_append": (INT, [VP, U64]),
    "fa_kv_table_address": (INT, [VP, U64, P(KvAddressC)]),
    "fa_kv_table_telemetry": (INT, [VP, P(KvTelemetryC)]),
    "fa_kv_table_reset": (INT, [VP]),
    "fa_kv_table_len": (U64, [VP]),
    "fa_kv_table_block_row": (INT, [VP, VP, U64, P(U64)]),
    "fa_paged_cache_create": (INT, [VP, U64, U64, U64, U64, INT, P(VP)]),
    "fa_paged_cache_destroy": (INT, [VP]),
    "fa_paged_cache_append": (INT, [VP, VP, VP, SZ, U64, P(RotaryC), P(U64)]),
    "fa_paged_cache_reset": (INT, [VP]),
    "fa_paged_cache_table": (VP, [VP]),
    "fa_paged_cache_k": (VP, [VP]),
    "fa_paged_cache_v": (VP, [VP]),
    "fa_paged_cache_bytes": (SZ, [VP]),
    "fa_paged_decode_prepare": (INT, [VP, VP, U64, VP, VP, U64, U64, U64, U64, U64, U64,
                                      P(ConfigC), F32, INT, P(VP)]),
    "fa_paged_decode_launch": (INT, [VP, VP, VP, SZ, VP, VP, SZ, VP, SZ]),
    "fa_paged_decode_plan_destroy": (INT, [VP]),
    "fa_paged_decode_plan_info": (INT, [VP, P(U64), P(U64), P(U64)]),
    "fa_paged_decode_plan_set_split": (INT, [VP, VP, U64]),
    "fa_paged_decode_noalloc": (INT, [VP, VP, U64, VP, VP, U64, U64, U64, U64, U64, U64,
                                      P(ConfigC),
                                      F32, INT, VP, SZ, VP, VP, SZ, VP, SZ]),
    "fa_paged_cache_decode": (INT, [VP, VP, VP, SZ, U64, P(ConfigC), F32, U64, VP, SZ]),
    "fa_forward_projection_variable": (INT, [VP, VP, SZ, VP, VP, SZ, VP, SZ, P(AsymmetricShapeC),
                                             P(VariableSequenceC), U64, P(ConfigC), F32, U64,
                                             INT]),
    "fa_resident_cache_create": (INT, [VP, U64, U64, U64, U64, INT, P(VP)]),
    "fa_resident_cache_destroy": (INT, [VP]),
    "fa_resident_cache_append": (INT, [VP, VP, VP, SZ, U64, P(U64)]),
    "fa_resident_cache_reset": (INT, [VP]),
    "fa_resident_cache_len": (U64, [VP]),
    "fa_resident_cache_k": (VP, [VP]),
    "fa_resident_cache_v": (VP, [VP]),
    "fa_resident_cache_bytes": (SZ, [VP]),
    "fa_resident_decode_prepare": (INT, [VP, U64, U64, U64, U64, U64, U64, P(ConfigC), F32, U64,
                                         INT, P(VP)]),
    "fa_resident_cache_decode": (INT, [VP, VP, VP, SZ, U64, P(ConfigC), F32, U64, VP, SZ]),
    "fa_chunked_prefill_paged_prepare": (INT, [VP, VP, U64, U64, U64, P(AsymmetricShapeC),
                                               P(ConfigC), P(AsymmetricRotaryC), INT, P(VP)]),
    "fa_chunked_prefill_paged_launch": (INT, [VP, VP, VP, SZ, VP, VP, SZ, VP, SZ]),
    "fa_prefill_plan_destroy": (INT, [VP]),
    "fa_paged_append_batched": (INT, [VP, VP, U64, VP, U64, U64, U64, U64, U64, U64, VP, VP, SZ,
                                      VP, VP, SZ, P(RotaryC), INT]),
    "fa_backward_grouped_layout": (INT, [P(GroupedShapeC), INT, P(BackwardLayoutC)]),
    "fa_backward_grouped_recompute": (INT, [VP, VP, SZ, VP, SZ, P(GroupedShapeC), P(ConfigC),
                                            INT]),
    "fa_backward_layout_mha": (INT, [P(AttentionShapeC), INT, P(BackwardLayoutC)]),
    "fa_backward_recompute_mha": (INT, [VP, VP, SZ, VP, SZ, P(AttentionShapeC), P(ConfigC),
                                        INT]),
    "fa_backward_grouped": (INT, [VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, P(GroupedShapeC),
                                  P(ConfigC), INT]),
    "fa_last_telemetry": (INT, [VP, P(TelemetryC)]),
    "fa_forward_gqa_rope_telemetry": (INT, [VP, P(GroupedShapeC), P(ConfigC), P(RotaryC), INT,
                                            P(TelemetryC)]),
    "fa_forward_mha_telemetry": (INT, [VP, P(AttentionShapeC), P(ConfigC), INT, P(TelemetryC)]),
    "fa_ctx_set_kernel_timing": (INT, [VP, I32]),
    "fa_ctx_pause_kernel_timing": (INT, [VP, I32]),
    "fa_ctx_set_prefill_precision": (INT, [VP, I32]),
    "fa_ctx_set_decode_policy": (INT, [VP, I32]),
    "fa_ctx_set_backward_policy": (INT, [VP, I32]),
    "fa_ctx_set_backward_kernel": (INT, [VP, I32]),
    "fa_device_record": (INT, [ctypes.c_char_p, ctypes.c_char_p, I32, I32, I32, ctypes.c_uint64,
                               ctypes.c_char_p, ctypes.c_size_t,
                               ctypes.POINTER(ctypes.c_uint64)]),
    "fa_ctx_kernel_timing": (INT, [VP, I32, P(ctypes.c_double), P(U64)]),
    "fa_ctx_kernel_timing_range": (INT, [VP, I32, P(ctypes.c_double), P(ctypes.c_double)]),
}


class FlatHipError(RuntimeError):
    """Typed error of a failed C-ABI call: ``variant`` names the reference enum variant."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.variant = STATUS.get(code, f"Unknown({code})")
        super().__init__(f"{self.variant}: {message}")


_lib = None


def lib():
    """Load the in-tree library. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `make -C flat-attention_amd` "
                "(or __graft_entry__.build()); there is no fallback implementation")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int):
    if rc != 0:
        msg = lib().fa_last_error_message()
        raise FlatHipError(rc, msg.decode() if msg else "")
