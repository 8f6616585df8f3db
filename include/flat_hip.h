/*
 * flat_hip.h — C ABI of the MI355X (gfx950 / CDNA4) backend for the FLAT-ATTENTION fused
 * attention hot path.
 *
 * The ABI replaces the roles of the reference crate's wgpu host executors. Every entry point
 * below names the reference surface it stands in for (file:line under the reference crate).
 * A Rust `hip_backend` module binds these symbols with `extern "C"` declarations; the Python
 * ctypes mirror in `flat-attention_amd/flat_attention_amd/` binds the same symbols for tests.
 *
 * Conventions
 *   - Every call returns an `int` status (`fa_status`). 0 is success. Non-zero codes map 1:1
 *     onto the reference's error enum variants; `fa_last_error_message()` returns the
 *     human-readable text (thread-local, same wording as the reference's Display impls).
 *   - Device pointers are plain `void*` obtained from `fa_buf_*` or from any HIP allocation on
 *     the context's device. Each device pointer is paired with its size in bytes so the library
 *     can reject undersized buffers before any launch (reference `BufferTooSmall`).
 *   - All work is enqueued on the context's single HIP stream. Only `fa_buf_download`,
 *     `fa_ctx_synchronize`, `fa_ctx_kernel_timing*`, the `*_host` convenience forwards and the
 *     destroy/free calls wait for it. Host metadata (block tables, work lists, per-sequence
 *     lengths) reaches the device by stream-ordered copies from pinned staging; a context cache
 *     that must grow is replaced without waiting (the old buffer is freed at context destroy).
 *     Prepared objects (`fa_prepare_*`, decode and paged-prefill plans) allocate at prepare
 *     time; their launches allocate nothing and copy nothing.
 *   - Validation always happens before any launch; nothing ever falls back to the CPU.
 *
 * Tensor layouts (element order, row-major):
 *   MHA / grouped:       Q,O [batch, q_heads, seq, head_dim]   K,V [batch, kv_heads, seq, head_dim]
 *   projection layout:   Q,O [batch, seq, q_heads*head_dim]    K,V [batch, seq, kv_heads*head_dim]
 *   paged pool:          K,V [physical_pages, page_size, kv_heads*head_dim]
 *   packed output:       [O (dtype) | LSE (f32)], LSE at byte offset round_up(O bytes, 4)
 *                        LSE is [batch, q_heads, query_len] (grouped and projection layouts).
 */
#ifndef FLAT_HIP_H
#define FLAT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 1

/* Status codes. Reference: FlatAttentionError src/lib.rs:362-380, WgpuFlatAttentionError
 * src/wgpu_backend.rs:39-100, PagedKvError src/paged_kv.rs:37-43, PagedDecodeError
 * src/wgpu_paged_decode.rs:28-70, WgpuChunkedProjectionPrefillError
 * src/wgpu_chunked_prefill.rs:40-52, WgpuPagedKvCacheError src/wgpu_paged_kv_cache.rs:15-33. */
typedef enum fa_status {
    FA_OK = 0,
    FA_ERR_ZERO_DIMENSION = 1,
    FA_ERR_SHAPE_OVERFLOW = 2,
    FA_ERR_INVALID_HEAD_GROUPING = 3,
    FA_ERR_INVALID_ROTARY_HEAD_DIM = 4,
    FA_ERR_INVALID_ROTARY_THETA = 5,
    FA_ERR_POSITION_OVERFLOW = 6,
    FA_ERR_LENGTH_MISMATCH = 7,
    FA_ERR_INVALID_SCALE = 8,
    FA_ERR_NON_FINITE_INPUT = 9,
    FA_ERR_UNAVAILABLE = 20,
    FA_ERR_UNSUPPORTED_HEAD_DIM = 21,
    FA_ERR_INDEX_SPACE_EXCEEDED = 22,
    FA_ERR_DISPATCH_LIMIT = 23,
    FA_ERR_BUFFER_TOO_SMALL = 24,
    FA_ERR_EMPTY_TABLE = 25,
    FA_ERR_TOO_MANY_MAPPED_PAGES = 26,
    FA_ERR_CAUSAL_VISIBILITY_MISMATCH = 27,
    FA_ERR_ZERO_QUERY_CHUNK_SIZE = 28,
    FA_ERR_UNSUPPORTED_DTYPE = 29,
    FA_ERR_INVALID_PAGE = 30,
    FA_ERR_EMPTY_CACHE = 31,          /* ResidentDecodeError::EmptyCache src/wgpu_decode.rs:105 */
    FA_ERR_INVALID_CACHE_LENGTH = 32, /* ResidentDecodeError::InvalidCacheLength :106 */
    FA_ERR_FOREIGN_BUFFER = 33,       /* WgpuFlatAttentionError::ForeignBuffer src/wgpu_backend.rs:56:
                                         a prepared object used with another context */
    FA_ERR_CANDIDATE_NOT_ENABLED = 34,        /* ExternalWgpuError::CandidateNotEnabled
                                               * src/wgpu_external.rs:62 */
    FA_ERR_UNSUPPORTED_CANDIDATE_SHAPE = 35,  /* ExternalWgpuError::UnsupportedCandidateShape :65 */
    FA_ERR_PAGED_ZERO_DIMENSION = 40,
    FA_ERR_CAPACITY_OVERFLOW = 41,
    FA_ERR_CAPACITY_EXCEEDED = 42,
    FA_ERR_GENERATION_OVERFLOW = 43,
    FA_ERR_NULL_ARGUMENT = 50,
    FA_ERR_HIP = 60,
    FA_ERR_SCRATCH_EXCEEDED = 61, /* no reference variant: fa_paged_decode_noalloc's scratch */
    FA_ERR_GRAPH_CAPTURE = 62     /* no reference variant: a call that allocates, uploads from the
                                     host, fills or waits while the stream is being captured */
} fa_status;

/* Storage dtype of Q/K/V/O. Math is always f32 (f32 online-softmax state, f32 accumulation);
 * LSE is always f32. Reference precedent: WgpuIoPrecision src/wgpu_f16_backend.rs:19. */
typedef enum fa_dtype { FA_DTYPE_F32 = 0, FA_DTYPE_F16 = 1, FA_DTYPE_BF16 = 2 } fa_dtype;

/* AttentionShape src/lib.rs:212. */
typedef struct fa_attention_shape {
    uint64_t batch, heads, seq_len, head_dim;
} fa_attention_shape;

/* GroupedAttentionShape src/grouped.rs:18. */
typedef struct fa_grouped_shape {
    uint64_t batch, q_heads, kv_heads, seq_len, head_dim;
} fa_grouped_shape;

/* AsymmetricGroupedAttentionShape src/asymmetric_grouped.rs:27. */
typedef struct fa_asymmetric_shape {
    uint64_t batch, q_heads, kv_heads, query_len, kv_len, head_dim, query_position_offset;
} fa_asymmetric_shape;

/* FlatAttentionConfig src/lib.rs:249 (softmax_scale: Option<f32> → has_softmax_scale flag). */
typedef struct fa_config {
    int32_t causal;
    int32_t has_softmax_scale;
    float softmax_scale;
} fa_config;

/* RotaryEmbeddingConfig src/rotary_grouped.rs:14. */
typedef struct fa_rotary {
    float theta;
    uint64_t position_offset;
} fa_rotary;

/* AsymmetricRotaryEmbeddingConfig src/projection_asymmetric.rs:19. */
typedef struct fa_asymmetric_rotary {
    float theta;
    uint64_t query_position_offset;
    uint64_t kv_position_offset;
} fa_asymmetric_rotary;

/* Packed [O|LSE] geometry. Mirrors PagedDecodeLayout src/wgpu_paged_decode.rs:18 and
 * WgpuResidentAttentionOutput src/wgpu_backend.rs:133. */
typedef struct fa_packed_layout {
    uint64_t output_elements;
    uint64_t lse_elements;
    uint64_t output_bytes;
    uint64_t lse_byte_offset;
    uint64_t combined_bytes;
} fa_packed_layout;

/* Kernel identities. Counterpart of RuntimeKernelId src/runtime_telemetry.rs:11 and
 * WgpuKernelVariant src/wgpu_backend.rs:31. */
typedef enum fa_kernel_id {
    FA_KERNEL_NONE = 0,
    FA_KERNEL_PREFILL_MFMA_BF16 = 1,      /* 32x32x16 bf16 MFMA, K rotated on load */
    FA_KERNEL_PREFILL_MFMA_F16 = 2,
    FA_KERNEL_PREFILL_MFMA_F32 = 3,       /* 32x32x2 f32 MFMA (f32 I/O contract) */
    FA_KERNEL_PREFILL_MFMA_BF16_PREROT = 4, /* K rotated once by a pre-pass */
    FA_KERNEL_PREFILL_MFMA_F16_PREROT = 5,
    FA_KERNEL_PREFILL_MFMA_F32_PREROT = 6,
    FA_KERNEL_DECODE_PAGED_SPLITK = 10,
    FA_KERNEL_DECODE_COMBINE = 11,
    FA_KERNEL_PAGED_APPEND = 12,
    FA_KERNEL_ROPE_TABLE = 13,
    FA_KERNEL_ROPE_ROTATE = 14,
    FA_KERNEL_DECODE_PAGED_MFMA = 15,     /* 16-bit KV, page_size % 16 == 0: P.V on MFMA */
    /* 16: retired (a transposed-V pre-pass that measured level) */
    FA_KERNEL_BACKWARD_RECOMPUTE = 17     /* delta + dK/dV + dQ recompute backward (MFMA) */
} fa_kernel_id;

/* RuntimeDispatchTelemetry src/runtime_telemetry.rs:159 + RuntimeTileGeometry :151 +
 * RuntimeDeviceFingerprint :35. Passive host metadata of the last logical call on a context. */
typedef struct fa_telemetry {
    int32_t kernel_id;            /* fa_kernel_id of the dominant (main) kernel */
    char kernel_name[64];
    uint32_t query_rows;          /* query rows per workgroup */
    uint32_t kv_rows;             /* K/V rows per inner tile */
    uint32_t workgroups[3];       /* grid of the main kernel */
    uint32_t workgroup_size;
    uint32_t dispatch_count;      /* kernel launches issued by the logical call */
    uint32_t temporary_allocation_count;
    uint64_t temporary_allocation_bytes;
    uint32_t splits;              /* split-K factor (decode), 1 otherwise */
    int32_t has_fallback_reason;
    char fallback_reason[128];
    char device_name[64];
    char device_arch[32];
    uint64_t device_fingerprint;  /* FNV-1a-64 of the canonical device record (fa_device_record) */
} fa_telemetry;

typedef struct fa_ctx fa_ctx;

/* ---------------------------------------------------------------- context ---------------
 * Replaces the owned-context constructors WgpuFlatAttention::new src/wgpu_backend.rs:177 and
 * WgpuRotaryGroupedAttention::new src/wgpu_rotary_grouped_backend.rs:78. Creates one HIP
 * stream on `device`; fails with FA_ERR_UNAVAILABLE when no gfx950 device is present. */
int fa_ctx_create(int device, fa_ctx** out);
int fa_ctx_destroy(fa_ctx* ctx);
/* HIP stream (hipStream_t) that every launch of this context is enqueued on. */
void* fa_ctx_stream(fa_ctx* ctx);
int fa_ctx_synchronize(fa_ctx* ctx);
/* adapter_name src/wgpu_backend.rs:337 */
int fa_ctx_device_name(fa_ctx* ctx, char* buf, size_t len);

const char* fa_status_string(int status);
const char* fa_last_error_message(void);
int fa_abi_version(void);

/* Resolved softmax scale: FlatAttentionConfig::resolved_scale src/lib.rs:257. */
int fa_resolved_scale(const fa_config* config, uint64_t head_dim, float* out);

/* ---------------------------------------------------------------- buffers ---------------
 * upload src/wgpu_backend.rs:465, download_attention :588. */
int fa_buf_alloc(fa_ctx* ctx, size_t bytes, void** out);
int fa_buf_free(fa_ctx* ctx, void* ptr);
int fa_buf_upload(fa_ctx* ctx, void* dst, const void* host, size_t bytes);
int fa_buf_download(fa_ctx* ctx, void* host, const void* src, size_t bytes);
int fa_buf_fill_u32(fa_ctx* ctx, void* dst, uint32_t value, size_t count);

/* ------------------------------------------------------------ packed layouts ------------ */
/* [O|LSE] geometry for `q_elements` output scalars of `dtype` and `lse_elements` f32. */
int fa_packed_layout_for(uint64_t output_elements, uint64_t lse_elements, int dtype,
                         fa_packed_layout* out);

/* ------------------------------------------------------------ prefill ------------------- */
/* WgpuFlatAttention::forward_resident src/wgpu_backend.rs:484 (MHA, [B,H,S,D]).
 * q,k,v: `dtype` tensors of shape->tensor_len elements; out_lse: packed [O|LSE]. */
int fa_forward_mha(fa_ctx* ctx, const void* q, const void* k, const void* v, size_t in_bytes,
                   void* out_lse, size_t out_bytes, const fa_attention_shape* shape,
                   const fa_config* config, int dtype);

/* WgpuRotaryGroupedAttention::forward_resident src/wgpu_rotary_grouped_backend.rs:163.
 * rotary == NULL runs plain GQA/MQA (forward_reference_grouped src/grouped.rs:81).
 * q_bytes / kv_bytes are the sizes of Q and of each of K, V. */
int fa_forward_gqa_rope(fa_ctx* ctx, const void* q, size_t q_bytes, const void* k,
                        const void* v, size_t kv_bytes, void* out_lse, size_t out_bytes,
                        const fa_grouped_shape* shape, const fa_config* config,
                        const fa_rotary* rotary, int dtype);

/* Prepared forward: PreparedGroupedForward::prepare src/wgpu_forward_grouped.rs:352 /
 * encode_prepared :496. prepare validates the buffers (Q, K, V, [O|LSE]), shape, config and
 * rotary exactly as fa_forward_gqa_rope does, resolves the kernel variant under the context's
 * current policies, and allocates what every launch needs: the RoPE (cos, sin) table for the
 * shape's positions (built on the context's stream) and the K rotation workspace. It may
 * allocate; it does not wait for the stream. fa_launch_prepared only enqueues kernels on the
 * context's stream (no allocation, copy or wait); a prepared forward used with another context
 * fails with FA_ERR_FOREIGN_BUFFER. Buffers stay bound: the caller keeps them alive and may
 * change their contents between launches. destroy waits for the stream, then frees. */
typedef struct fa_prepared_forward fa_prepared_forward;
int fa_prepare_gqa_rope(fa_ctx* ctx, const void* q, size_t q_bytes, const void* k,
                        const void* v, size_t kv_bytes, void* out_lse, size_t out_bytes,
                        const fa_grouped_shape* shape, const fa_config* config,
                        const fa_rotary* rotary, int dtype, fa_prepared_forward** out);
int fa_prepare_mha(fa_ctx* ctx, const void* q, const void* k, const void* v, size_t in_bytes,
                   void* out_lse, size_t out_bytes, const fa_attention_shape* shape,
                   const fa_config* config, int dtype, fa_prepared_forward** out);
int fa_launch_prepared(fa_ctx* ctx, const fa_prepared_forward* prepared);
int fa_prepared_forward_layout(const fa_prepared_forward* prepared, fa_packed_layout* out);
int fa_prepared_forward_destroy(fa_prepared_forward* prepared);

/* Owned-context host forwards: WgpuFlatAttention::forward src/wgpu_backend.rs:445 and
 * WgpuRotaryGroupedAttention::forward src/wgpu_rotary_grouped_backend.rs:117. Inputs are
 * validated on the host (length and finiteness, reference validate_input src/lib.rs:428),
 * uploaded, run and read back. Host data is in `dtype` storage; output O in `dtype`, LSE f32. */
int fa_forward_mha_host(fa_ctx* ctx, const void* q, const void* k, const void* v,
                        uint64_t q_len, uint64_t k_len, uint64_t v_len,
                        const fa_attention_shape* shape, const fa_config* config, int dtype,
                        void* out, float* lse);
int fa_forward_gqa_rope_host(fa_ctx* ctx, const void* q, const void* k, const void* v,
                             uint64_t q_len, uint64_t k_len, uint64_t v_len,
                             const fa_grouped_shape* shape, const fa_config* config,
                             const fa_rotary* rotary, int dtype, void* out, float* lse);

/* Rectangular projection-layout GQA + RoPE with a causal query offset:
 * ExternalAsymmetricProjectionRotaryGroupedPipeline::encode src/wgpu_external_asymmetric.rs:192
 * (rotate_k = 1) and encode_pre_rotated_k :203 (rotate_k = 0). rotary == NULL: no RoPE. */
int fa_forward_projection_asymmetric(fa_ctx* ctx, const void* q, size_t q_bytes,
                                     const void* k, const void* v, size_t kv_bytes,
                                     void* out_lse, size_t out_bytes,
                                     const fa_asymmetric_shape* shape, const fa_config* config,
                                     const fa_asymmetric_rotary* rotary, int32_t rotate_k,
                                     int dtype);

/* ExternalAsymmetricProjectionRotaryGroupedPipeline::encode_pre_rotated_k_decode_kv_reuse
 * src/wgpu_external_asymmetric.rs:216 (the opt-in M48 candidate): q_len = 1 decode over
 * pre-rotated K in projection layout, each K/V tile read once for every query head of its GQA
 * group. Fails with FA_ERR_UNSUPPORTED_CANDIDATE_SHAPE unless query_len == 1 and
 * q_heads / kv_heads >= 2, then checks as fa_forward_projection_asymmetric. Q is rotated at
 * rotary->query_position_offset; causal masking keeps keys <= shape->query_position_offset.
 * Output [O | LSE] as for fa_forward_projection_asymmetric. Runs through the allocation-free
 * decode (fa_paged_decode_noalloc, each batch element one page of kv_len rows): no allocation
 * and no wait for the stream per token. A shape whose work lists or partials exceed that
 * scratch prepares, launches and releases a one-call decode plan instead (allocates, and waits
 * for the stream when releasing it). Refused with FA_ERR_GRAPH_CAPTURE while capturing. */
int fa_forward_projection_asymmetric_decode_kv_reuse(fa_ctx* ctx, const void* q, size_t q_bytes,
                                                     const void* k, const void* v,
                                                     size_t kv_bytes, void* out_lse,
                                                     size_t out_bytes,
                                                     const fa_asymmetric_shape* shape,
                                                     const fa_config* config,
                                                     const fa_asymmetric_rotary* rotary,
                                                     int dtype);

/* WgpuChunkedProjectionPrefillPipeline::encode src/wgpu_chunked_prefill.rs:156: full-sequence
 * projection-layout GQA + RoPE prefill whose query rows are processed in chunks of
 * `query_chunk_size` with absolute causal and RoPE positions. Output is identical for every
 * chunk size. */
int fa_chunked_prefill(fa_ctx* ctx, const void* q, size_t q_bytes, const void* k,
                       const void* v, size_t kv_bytes, void* out_lse, size_t out_bytes,
                       const fa_grouped_shape* shape, const fa_config* config,
                       const fa_rotary* rotary, uint64_t query_chunk_size, int dtype);

/* ------------------------------------------------------------ paged KV table ------------
 * PagedKvTable src/paged_kv.rs:76 (host metadata only). */
typedef struct fa_kv_table fa_kv_table;
typedef struct fa_kv_address {
    uint64_t physical_page, offset_in_page, generation;
} fa_kv_address;
typedef struct fa_kv_telemetry {  /* PagedKvTelemetry src/paged_kv.rs:28 */
    uint64_t live_tokens, capacity_tokens, mapped_pages, free_pages,
        internal_fragmentation_tokens, generation;
} fa_kv_telemetry;

int fa_kv_table_create(uint64_t page_size, uint64_t physical_pages, fa_kv_table** out);
int fa_kv_table_destroy(fa_kv_table* t);
int fa_kv_table_clone(const fa_kv_table* t, fa_kv_table** out);
int fa_kv_table_append(fa_kv_table* t, uint64_t tokens);     /* append :113 */
/* address :143 — returns FA_OK and fills `out`, or FA_ERR_EMPTY_TABLE when unmapped. */
int fa_kv_table_address(const fa_kv_table* t, uint64_t logical_token, fa_kv_address* out);
int fa_kv_table_telemetry(const fa_kv_table* t, fa_kv_telemetry* out); /* telemetry :160 */
int fa_kv_table_reset(fa_kv_table* t);                        /* reset :176 */
uint64_t fa_kv_table_len(const fa_kv_table* t);
/* WgpuPagedKvTable::from_table src/wgpu_paged_decode.rs:162: flattens the live logical pages
 * to physical page ids. `*count` receives the number of mapped pages. */
int fa_kv_table_block_row(const fa_kv_table* t, int32_t* out, uint64_t capacity,
                          uint64_t* count);

/* ------------------------------------------------------------ paged KV cache ------------
 * WgpuPagedKvCache src/wgpu_paged_kv_cache.rs:76. Device storage
 * [physical_pages, page_size, kv_heads*head_dim] in `dtype` for K and V, plus a table. */
typedef struct fa_paged_cache fa_paged_cache;
int fa_paged_cache_create(fa_ctx* ctx, uint64_t page_size, uint64_t physical_pages,
                          uint64_t kv_heads, uint64_t head_dim, int dtype,
                          fa_paged_cache** out);                   /* new :99 */
int fa_paged_cache_destroy(fa_paged_cache* cache);
/* record_append :206. Sources are device [append_len, kv_heads*head_dim] rows. K must already
 * be RoPE-rotated (reference contract :73) unless `rotate_k` is non-NULL, in which case rows are
 * rotated at positions rotate_k->position_offset + live_len + i while they are scattered. */
int fa_paged_cache_append(fa_paged_cache* cache, const void* k_src, const void* v_src,
                          size_t src_bytes, uint64_t append_len, const fa_rotary* rotate_k,
                          uint64_t* new_len);
int fa_paged_cache_reset(fa_paged_cache* cache);                  /* reset */
const fa_kv_table* fa_paged_cache_table(const fa_paged_cache* cache); /* table */
void* fa_paged_cache_k(fa_paged_cache* cache);                    /* k_buffer */
void* fa_paged_cache_v(fa_paged_cache* cache);                    /* v_buffer */
size_t fa_paged_cache_bytes(const fa_paged_cache* cache);          /* bytes of K (= of V) */

/* ------------------------------------------------------------ paged decode --------------
 * WgpuPagedDecodePipeline::encode src/wgpu_paged_decode.rs:300 generalised to a batch of
 * sequences over one shared page pool. Prepare validates the host block tables (every entry a
 * valid physical page, coverage of each context, causal visibility q_position + 1 >= ctx_len)
 * and makes them resident; launch enqueues the split-K kernel plus the LSE combine.
 *   block_tables: [n_seqs, max_pages] int32 physical page ids (host)
 *   ctx_lens:     [n_seqs] live tokens per sequence (host)
 *   q_positions:  [n_seqs] RoPE position of each query, NULL → ctx_len - 1
 *   q:            [n_seqs, q_heads*head_dim], out_lse: [O n_seqs*q_heads*head_dim | LSE n_seqs*q_heads]
 */
typedef struct fa_decode_plan fa_decode_plan;
int fa_paged_decode_prepare(fa_ctx* ctx, const int32_t* block_tables, uint64_t max_pages,
                            const int32_t* ctx_lens, const int32_t* q_positions,
                            uint64_t n_seqs, uint64_t page_size, uint64_t physical_pages,
                            uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                            const fa_config* config, float theta, int dtype,
                            fa_decode_plan** out);
int fa_paged_decode_launch(fa_ctx* ctx, const fa_decode_plan* plan, const void* q,
                           size_t q_bytes, const void* k_pool, const void* v_pool,
                           size_t pool_bytes, void* out_lse, size_t out_bytes);
int fa_paged_decode_plan_destroy(fa_decode_plan* plan);
/* Longest split-K segment (tokens), number of (segment, unit) work items, where a unit is
 * (kv head, chunk of <= 16 query heads), and the partials workspace in bytes. */
int fa_paged_decode_plan_info(const fa_decode_plan* plan, uint64_t* split_tokens,
                              uint64_t* work_items, uint64_t* workspace_bytes);
/* Override tokens per split (multiple of 16; 0 = automatic) before launch. Tests use this to
 * check split invariance. */
int fa_paged_decode_plan_set_split(fa_ctx* ctx, fa_decode_plan* plan, uint64_t split_tokens);

/* Allocation-free paged decode. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid hipMalloc). It uploads
 * its host-built work list on every call, so it is not for graph capture (capture a prepared
 * plan's fa_paged_decode_launch with fa_graph_* instead). Same arguments, validation and results (bitwise) as
 * fa_paged_decode_prepare followed by fa_paged_decode_launch with the automatic split, in one
 * call that allocates no device or pinned host memory: the block tables, lengths, query
 * positions, work list, the queries' RoPE (cos, sin) rows and the split-K partials live in a
 * static per-device scratch array of 64 MiB (4 MiB of it for tables and work lists), which each
 * GPU holds until the process ends. A call needing more fails with FA_ERR_SCRATCH_EXCEEDED
 * before any device work. The metadata reaches the scratch by a stream-ordered copy from a
 * host area owned by the context; a call waits only until the previous call's copy has left
 * that area. Every call on one GPU shares that GPU's scratch; calls from different contexts
 * (streams) are ordered on the GPU: each call makes its stream wait for the event the previous
 * call on that GPU recorded after its kernels, and records its own (no host wait, no
 * allocation). Refused with FA_ERR_GRAPH_CAPTURE while the context's stream is captured (the
 * metadata copy would read a host area that later calls rewrite). */
int fa_paged_decode_noalloc(fa_ctx* ctx, const int32_t* block_tables, uint64_t max_pages,
                            const int32_t* ctx_lens, const int32_t* q_positions, uint64_t n_seqs,
                            uint64_t page_size, uint64_t physical_pages, uint64_t q_heads,
                            uint64_t kv_heads, uint64_t head_dim, const fa_config* config,
                            float theta, int dtype, const void* q, size_t q_bytes,
                            const void* k_pool, const void* v_pool, size_t pool_bytes,
                            void* out_lse, size_t out_bytes);

/* Single-sequence convenience mirror of WgpuPagedDecodePipeline::encode: decode one query
 * vector over `cache` at `q_rope_position`. */
int fa_paged_cache_decode(fa_ctx* ctx, const fa_paged_cache* cache, const void* q,
                          size_t q_bytes, uint64_t q_heads, const fa_config* config,
                          float theta, uint64_t q_rope_position, void* out_lse,
                          size_t out_bytes);

/* ------------------------------------------------------------ variable-length prefill ----
 * ExternalVariableProjectionRotaryGroupedPipeline::encode src/wgpu_external_variable.rs:138 (M12).
 * Q [batch, shape->query_len, q_heads*head_dim], K/V [batch, shape->kv_len, kv_heads*head_dim] are
 * padded projection-layout tensors (shape->query_position_offset is ignored); meta[b] gives the
 * active extents and query origins of sequence b (VariableLengthSequenceMetadata :25). Sequence b
 * attends over its first active_kv_len K/V rows only (padded rows are never read), causally at
 * query_position_offset + t; Q is rotated at query_rope_position_offset + t, K at
 * kv_position_offset + key (VariableLengthRotaryEmbeddingConfig :40). Output [O | LSE] as for
 * fa_forward_projection_asymmetric; padded query rows get O = 0 and LSE = -inf. Errors follow
 * validate_dispatch :229 (LengthMismatch for the metadata count and for active lengths above the
 * padded ones, PositionOverflow past the i32 position space); there is no batch limit. */
typedef struct fa_variable_sequence {
    uint64_t active_query_len, active_kv_len, query_position_offset, query_rope_position_offset;
} fa_variable_sequence;
int fa_forward_projection_variable(fa_ctx* ctx, const void* q, size_t q_bytes, const void* k,
                                   const void* v, size_t kv_bytes, void* out_lse,
                                   size_t out_bytes, const fa_asymmetric_shape* shape,
                                   const fa_variable_sequence* meta, uint64_t n_meta,
                                   const fa_config* config, float theta,
                                   uint64_t kv_position_offset, int dtype);

/* ------------------------------------------------------------ resident KV cache ---------
 * WgpuResidentKvCache src/wgpu_kv_cache.rs:79: fixed-capacity K and V storage
 * [batch, capacity, kv_heads*head_dim] in `dtype`, one live length shared by the batch. */
typedef struct fa_resident_cache fa_resident_cache;
int fa_resident_cache_create(fa_ctx* ctx, uint64_t batch, uint64_t kv_heads, uint64_t capacity,
                             uint64_t head_dim, int dtype, fa_resident_cache** out); /* new :104 */
int fa_resident_cache_destroy(fa_resident_cache* cache);
/* record_append :212. Sources are device [batch, append_len, kv_heads*head_dim]; K is already
 * RoPE-rotated (the decode contract). Rows land after the live prefix of every batch element;
 * FA_ERR_CAPACITY_EXCEEDED when len + append_len > capacity. */
int fa_resident_cache_append(fa_resident_cache* cache, const void* k_src, const void* v_src,
                             size_t src_bytes, uint64_t append_len, uint64_t* new_len);
int fa_resident_cache_reset(fa_resident_cache* cache);               /* reset :200 */
uint64_t fa_resident_cache_len(const fa_resident_cache* cache);       /* len :174 */
void* fa_resident_cache_k(fa_resident_cache* cache);                  /* k_buffer :189 */
void* fa_resident_cache_v(fa_resident_cache* cache);                  /* v_buffer :194 */
size_t fa_resident_cache_bytes(const fa_resident_cache* cache);        /* bytes of K (= of V) */

/* ------------------------------------------------------------ resident decode -----------
 * WgpuResidentDecodePipeline::encode_external_pre_rotated_k src/wgpu_decode.rs:301: q_len = 1
 * decode of `batch` queries over framework-owned fixed-capacity K (pre-rotated) and V
 * [batch, capacity, kv_heads*head_dim], kv_len live rows each, Q rotated at q_rope_position.
 * Validation follows the reference (causal visibility, zero dimensions, EmptyCache,
 * InvalidCacheLength, head_dim, head grouping, theta, scale). The returned plan launches with
 * fa_paged_decode_launch(ctx, plan, q, q_bytes, k, v, kv_bytes, out_lse, out_bytes): the layout
 * is a page pool with one `capacity`-row page per batch element. Output [O | LSE] as for paged
 * decode (batch*q_heads rows). */
int fa_resident_decode_prepare(fa_ctx* ctx, uint64_t batch, uint64_t capacity, uint64_t kv_len,
                               uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                               const fa_config* config, float theta, uint64_t q_rope_position,
                               int dtype, fa_decode_plan** out);
/* WgpuResidentDecodePipeline::encode src/wgpu_decode.rs:265: decode over a resident cache's live
 * rows (prepares, launches and releases a plan; waits for the stream when releasing). */
int fa_resident_cache_decode(fa_ctx* ctx, const fa_resident_cache* cache, const void* q,
                             size_t q_bytes, uint64_t q_heads, const fa_config* config,
                             float theta, uint64_t q_rope_position, void* out_lse,
                             size_t out_bytes);

/* ------------------------------------------------------------ recompute backward -------- */
/* WgpuGroupedBackwardRecomputeLayout src/wgpu_backward_grouped.rs:17-56: the packed contract
 * Q|K|V|dO|O|LSE (forward side) and dQ|dK|dV (gradients). Q, dO, O, dQ hold
 * [batch, q_heads, seq, head_dim], K, V, dK, dV [batch, kv_heads, seq, head_dim] (native KV-head
 * cardinality), LSE [batch, q_heads, seq]. Tensors are `dtype` elements, LSE is f32; offsets and
 * sizes here are in BYTES (for f32 they are the reference's element offsets times 4). */
typedef struct fa_backward_layout {
    uint64_t q_elements, kv_elements, lse_elements;
    uint64_t packed_forward_bytes, gradient_bytes;
    uint64_t q_offset, k_offset, v_offset, d_out_offset, output_offset, lse_offset;
    uint64_t dq_offset, dk_offset, dv_offset;
} fa_backward_layout;
/* WgpuGroupedBackwardRecomputePipeline::layout src/wgpu_backward_grouped.rs:181 */
int fa_backward_grouped_layout(const fa_grouped_shape* shape, int dtype, fa_backward_layout* out);
/* WgpuGroupedBackwardRecomputePipeline::encode src/wgpu_backward_grouped.rs:318 (prepare :231 +
 * encode_prepared :302): dQ, dK, dV recomputed from the packed forward buffer into the packed
 * gradient buffer (shaders/flat_backward_grouped_recompute.wgsl; CPU oracle
 * backward_reference_grouped src/backward_grouped.rs:17). Buffer sizes are checked against the
 * layout (FA_ERR_BUFFER_TOO_SMALL). Deterministic: every gradient element has one writer. */
int fa_backward_grouped_recompute(fa_ctx* ctx, const void* packed_forward, size_t forward_bytes,
                                  void* packed_grads, size_t grads_bytes,
                                  const fa_grouped_shape* shape, const fa_config* config,
                                  int dtype);
/* M18 canonical MHA form: WgpuBackwardRecomputePipeline::layout src/wgpu_backward.rs:162 and
 * encode :201 (packing pack_backward_recompute_inputs :282) — the grouped backward with
 * kv_heads == heads; the fa_backward_layout fields are filled the same way (q_elements ==
 * kv_elements = tensor_elements). */
int fa_backward_layout_mha(const fa_attention_shape* shape, int dtype, fa_backward_layout* out);
int fa_backward_recompute_mha(fa_ctx* ctx, const void* packed_forward, size_t forward_bytes,
                              void* packed_grads, size_t grads_bytes,
                              const fa_attention_shape* shape, const fa_config* config, int dtype);
/* The same backward over separate tensors (e.g. O|LSE straight from fa_forward_gqa_rope's packed
 * output): q, d_out, out, dq hold q_elements, k, v, dk, dv kv_elements, lse lse_elements. */
int fa_backward_grouped(fa_ctx* ctx, const void* q, const void* k, const void* v,
                        const void* d_out, const void* out, const float* lse, void* dq, void* dk,
                        void* dv, const fa_grouped_shape* shape, const fa_config* config,
                        int dtype);

/* ------------------------------------------------------------ chunked prefill (paged) ---
 * Chunked prefill whose K/V live in the shared page pool: the chunk's queries
 * [batch, query_len, q_heads*head_dim] attend causally (query i at absolute position
 * query_position_offset + i) over kv_len live tokens of each sequence's block table.
 * K in the pool is pre-rotated; Q is rotated at rotary->query_position_offset + i.
 * Follows forward_reference_projection_grouped_rope_chunked_prefill
 * src/chunked_projection_prefill.rs:63 with the K/V source of WgpuPagedKvCache. */
typedef struct fa_prefill_plan fa_prefill_plan;
int fa_chunked_prefill_paged_prepare(fa_ctx* ctx, const int32_t* block_tables,
                                     uint64_t max_pages, uint64_t page_size,
                                     uint64_t physical_pages, const fa_asymmetric_shape* shape,
                                     const fa_config* config, const fa_asymmetric_rotary* rotary,
                                     int dtype, fa_prefill_plan** out);
int fa_chunked_prefill_paged_launch(fa_ctx* ctx, const fa_prefill_plan* plan, const void* q,
                                    size_t q_bytes, const void* k_pool, const void* v_pool,
                                    size_t pool_bytes, void* out_lse, size_t out_bytes);
int fa_prefill_plan_destroy(fa_prefill_plan* plan);

/* Batched paged append with RoPE-on-append (record_append src/wgpu_paged_kv_cache.rs:206 for a
 * batch of sequences): rows i of sequence s, from [n_seqs, append_len, kv_heads*head_dim]
 * sources, land at logical token start_lens[s] + i of that sequence's block table. K rows are
 * rotated at position rotary->position_offset + start_lens[s] + i when rotary != NULL.
 * block_tables [n_seqs, max_pages] and start_lens [n_seqs] are host arrays, validated (page ids,
 * capacity) before anything is enqueued; the call returns once the scatter has completed. */
int fa_paged_append_batched(fa_ctx* ctx, const int32_t* block_tables, uint64_t max_pages,
                            const int32_t* start_lens, uint64_t n_seqs, uint64_t append_len,
                            uint64_t page_size, uint64_t physical_pages, uint64_t kv_heads,
                            uint64_t head_dim, const void* k_src, const void* v_src,
                            size_t src_bytes, void* k_pool, void* v_pool, size_t pool_bytes,
                            const fa_rotary* rotary, int dtype);

/* ------------------------------------------------------------ telemetry ------------------
 * runtime_telemetry src/wgpu_backend.rs:374: metadata of the last logical call on `ctx`. */
int fa_last_telemetry(fa_ctx* ctx, fa_telemetry* out);
/* ------------------------------------------------------------ HIP graphs -----------------
 * No counterpart in the reference (its callers record passes into a wgpu command encoder and
 * submit it; these are the HIP form of that for launch-bound loops). capture_begin starts a
 * thread-local capture of the context's stream; the launches that follow are recorded, not
 * run, until capture_end turns them into an executable graph that fa_graph_launch replays on
 * the stream (same buffers, same arguments; the caller changes buffer contents between
 * replays). Only launches that enqueue kernels alone may be captured: prepared plans
 * (fa_paged_decode_launch, fa_launch_prepared, fa_chunked_prefill_paged_launch,
 * fa_backward_launch_prepared) and one-shot calls whose context caches are already sized. While
 * capturing, a call that would allocate device memory, upload host data, fill a buffer or wait
 * for the stream fails with FA_ERR_GRAPH_CAPTURE and enqueues nothing; per-kernel timing
 * events are not recorded. */
typedef struct fa_graph fa_graph;
int fa_graph_capture_begin(fa_ctx* ctx);
int fa_graph_capture_end(fa_ctx* ctx, fa_graph** out);
int fa_graph_launch(fa_ctx* ctx, const fa_graph* graph);
int fa_graph_destroy(fa_graph* graph);

/* Passive telemetry snapshot: WgpuFlatAttention::runtime_telemetry src/wgpu_backend.rs (M29,
 * tests/m29_runtime_telemetry.rs:7): the record a one-shot fa_forward_gqa_rope / fa_forward_mha
 * of this shape would leave in fa_last_telemetry (kernel, geometry, dispatch count, the
 * allocations the context's caches would still need, fallback reason), built on the host from
 * the same decisions without device work, allocation or synchronisation. Shape, rotary and
 * dtype errors as for the forward; buffers are not involved. */
int fa_forward_gqa_rope_telemetry(fa_ctx* ctx, const fa_grouped_shape* shape,
                                  const fa_config* config, const fa_rotary* rotary, int dtype,
                                  fa_telemetry* out);
int fa_forward_mha_telemetry(fa_ctx* ctx, const fa_attention_shape* shape,
                             const fa_config* config, int dtype, fa_telemetry* out);

/* Variant selection policy. kernel_variant_for_head_dim src/wgpu_backend.rs:430.
 * prerotate_k: 0 = rotate K tiles on load inside the prefill kernel, 1 = rotate K once in a
 * pre-pass, -1 = automatic (default). */
int fa_ctx_set_prefill_policy(fa_ctx* ctx, int32_t prerotate_k);
/* Main loop of the 16-bit contiguous prefill (kernel-variant selection, the role of
 * WgpuKernelVariant src/wgpu_backend.rs:31-37): -1 (default) and 1 the assembly kernel
 * fa_prefill_a64_bf16 / fa_prefill_a64_f16 (64 query rows per wave, persistent grid) where it
 * applies: bf16 or f16 storage, head_dim 128, RoPE with K rotated by the pre-pass, power-of-two
 * GQA group, 16-byte aligned rows (the precise-score mode: bf16 only); 0 the
 * HIP kernels only. Other inputs always run the HIP kernels. Both give results within the same
 * tolerance of the oracle (not bitwise equal: the assembly kernel scales Q by scale * log2 e
 * before its one rounding to bf16); the telemetry's kernel name says which ran. */
int fa_ctx_set_prefill_kernel(fa_ctx* ctx, int32_t assembly);
/* Score precision of the 16-bit RoPE prefill (the NumericalMode choice of src/numerical.rs:18,
 * applied to this backend). 0 (default): the rotated Q and K are rounded to the storage type
 * before Q.K^T, so a score s carries a relative error up to about 2^-8 (bf16) -- within the
 * 2e-2 bar for unit-scale inputs, not for scores of tens. 1: the rotated Q and K keep their
 * 16-bit residuals and each score block takes three MFMAs (f32-level scores, about 0.6x the
 * default's throughput where the assembly kernel runs: bf16, head_dim 128, power-of-two group,
 * with K and its residual written by a split pre-rotation pass; elsewhere the HIP kernel
 * rotates K on load, about 0.3x). Applies to contiguous K that the call rotates;
 * K that is stored rotated (paged cache, pre-rotated asymmetric input) is used as stored.
 * Other values: FA_ERR_UNAVAILABLE. */
int fa_ctx_set_prefill_precision(fa_ctx* ctx, int32_t mode);
/* Decode work layout, read when a decode plan is prepared (kernel_variant_for_head_dim
 * src/wgpu_backend.rs:430 generalised). grouped: -1 = automatic (default: 16-bit KV with
 * page_size % 16 == 0, automatic split and <= 8 KV-head units run head-grouped workgroups),
 * 0 = one-wave workgroups for every plan; 1 = the same as -1. */
int fa_ctx_set_decode_policy(fa_ctx* ctx, int32_t grouped);
/* dQ policy of the recompute backward (no counterpart in the reference, whose backward
 * recomputes every product per scalar gradient, src/wgpu_backward_grouped.rs:318). store_ds:
 * -1 = automatic (default) and 1: with 16-bit storage and 16-byte aligned tensors, bwd_dkdv also
 * writes dS (2 bytes per (query, key) pair of every visible 32 x 32 block, kept in a context
 * workspace, used when it fits in 2 GiB) and dQ = dS K reads it back; 0 = dQ recomputes S and dP
 * (no workspace). Both are deterministic and use the same dS values up to MFMA summation order. */
int fa_ctx_set_backward_policy(fa_ctx* ctx, int32_t store_ds);
/* dK/dV kernel of the recompute backward (kernel-variant selection, the role of
 * WgpuKernelVariant src/wgpu_backend.rs:31-37 for the backward of src/wgpu_backward_grouped.rs:
 * 181-329): -1 (default) and 1 the assembly kernel fa_bwd_dkdv_a64_bf16 where it applies: bf16,
 * head_dim 128, seq_len a multiple of 128, dS stored (fa_ctx_set_backward_policy), 16-byte
 * aligned tensors; 0 the HIP kernel only. Both are within the same tolerance of the oracle (not
 * bitwise equal: the assembly kernel adds -LSE / scale and -delta through the MFMA accumulator
 * inputs, a different f32 summation order); the telemetry's kernel name says which ran
 * (bwd_dkdv_a64). */
int fa_ctx_set_backward_kernel(fa_ctx* ctx, int32_t assembly);
int fa_kernel_variant_for_shape(fa_ctx* ctx, uint64_t head_dim, int32_t has_rope, int dtype,
                                int32_t* kernel_id);

/* RuntimeDeviceFingerprint::{canonical_record, stable_fingerprint} src/runtime_telemetry.rs:49-67
 * (escape_component :70, fnv1a64 :83): the device record behind fa_telemetry::device_fingerprint,
 * "name=..;arch=..;driver=..;cus=..;clock_khz=..;mem=.." with '%', ';' and '=' inside values
 * escaped as %25, %3b and %3d, and its FNV-1a-64 hash. The fields are this build's (the HIP
 * device properties), not the WGPU adapter's. Writes the record (truncated to cap - 1 bytes,
 * NUL-terminated) when out is not null. Pure host code. */
int fa_device_record(const char* name, const char* arch, int32_t driver, int32_t cus,
                     int32_t clock_khz, uint64_t mem_bytes, char* out, size_t cap,
                     uint64_t* fingerprint);

/* Per-kernel device timing (extends runtime_telemetry src/wgpu_backend.rs:374, which carries no
 * durations). While enabled, every dispatch the context issues is bracketed by HIP events on
 * the context's stream. Enabling (or disabling) clears the accumulated totals. */
int fa_ctx_set_kernel_timing(fa_ctx* ctx, int32_t enable);
/* Pauses (paused != 0) or resumes per-dispatch timing without waiting for the stream and
 * without clearing the totals: dispatches issued while paused carry no events. Lets a caller
 * time whole operations (its own events, no per-kernel events inside) and their kernels in
 * alternate steps of one run. No effect while timing is disabled. */
int fa_ctx_pause_kernel_timing(fa_ctx* ctx, int32_t paused);
/* Waits for the context's stream, then returns the summed duration (ms) and the number of
 * timed dispatches of `kernel_id` (an fa_kernel_id naming one kernel: a prefill variant id
 * names the prefill kernel alone, FA_KERNEL_ROPE_ROTATE the K pre-rotation pass,
 * FA_KERNEL_DECODE_PAGED_SPLITK / _MFMA the split kernel and FA_KERNEL_DECODE_COMBINE the
 * combine) since timing was enabled. */
int fa_ctx_kernel_timing(fa_ctx* ctx, int32_t kernel_id, double* total_ms, uint64_t* launches);
/* Shortest and longest single timed dispatch (ms) of `kernel_id` since timing was enabled
 * (0 when none ran); waits for the context's stream like fa_ctx_kernel_timing. */
int fa_ctx_kernel_timing_range(fa_ctx* ctx, int32_t kernel_id, double* min_ms, double* max_ms);

#ifdef __cplusplus
}
#endif

#endif /* FLAT_HIP_H */
