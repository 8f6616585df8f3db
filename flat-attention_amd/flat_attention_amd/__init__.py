"""MI355X (gfx950) backend for the FLAT-ATTENTION fused attention hot path.

The compute lives in ``libflat_hip.so`` (hand-written HIP kernels + C ABI, see
``include/flat_hip.h``); this package is the host-side mirror of the reference crate's
executor API over that ABI. Importing it does not load the library; the first call does,
and fails loudly when it has not been built.
"""

from ._lib import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, LIB_PATH, FlatHipError, lib)
from .api import (AsymmetricGroupedAttentionShape, AsymmetricRotaryEmbeddingConfig,
                  AttentionShape, DeviceBuffer, FlatAttentionConfig, FlatAttentionOutput,
                  GroupedAttentionShape, HipAsymmetricProjectionPipeline,
                  HipChunkedProjectionPrefillPipeline, HipContext, HipFlatAttention, HipGraph,
                  HipPagedDecodePipeline, HipPagedKvCache, HipProjectionRotaryGroupedPipeline, HipResidentDecodePipeline,
                  HipResidentKvCache, HipRotaryGroupedAttention, ResidentDecodePlan,
                  PackedLayout, PagedChunkedPrefillPlan, PagedDecodePlan, PagedKvAddress,
                  PagedKvConfig, PagedKvTable, PagedKvTelemetry, RotaryEmbeddingConfig,
                  RuntimeDispatchTelemetry, HipVariableProjectionPipeline,
                  VariableLengthRotaryEmbeddingConfig, VariableLengthSequenceMetadata,
                  FlatAttentionBackwardOutput, GroupedBackwardRecomputeLayout,
                  HipGroupedBackwardRecomputePipeline, PreparedGroupedBackwardRecompute,
                  PreparedGroupedForward,
                  grouped_backward_layout, pack_grouped_backward_recompute_inputs,
                  HipBackwardRecomputePipeline, pack_backward_recompute_inputs,
                  bf16_bits_to_f32, download_attention,
                  f32_to_bf16_bits, host_storage, packed_layout, paged_append_batched,
                  paged_decode_noalloc,
                  storage_np_dtype, storage_to_f32)

__all__ = [n for n in dir() if not n.startswith("_")]
