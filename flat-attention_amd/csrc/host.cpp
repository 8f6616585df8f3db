// C-ABI host layer of the gfx950 FLAT-ATTENTION backend (include/flat_hip.h).
//
// Validation restates the reference's host-side checks before anything is enqueued
// (AttentionShape::validate src/lib.rs:236, GroupedAttentionShape::validate src/grouped.rs:57,
// RotaryEmbeddingConfig::validate src/rotary_grouped.rs:22, resolved_scale src/lib.rs:257,
// WgpuPagedDecodePipeline::encode src/wgpu_paged_decode.rs:300-359, PagedKvTable
// src/paged_kv.rs:84-188, WgpuPagedKvCache::record_append src/wgpu_paged_kv_cache.rs:206-280).
// Errors are returned as fa_status codes with the reference's message text; nothing falls back
// to a CPU path.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "../../include/flat_hip.h"
#include "kernels.hpp"

using fa::Dtype;

// ---------------------------------------------------------------------------- errors
namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int ok() {
    g_error.clear();
    return FA_OK;
}

#define HIP_TRY(expr)                                                                       \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return fail(FA_ERR_HIP, "HIP call %s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

constexpr uint64_t kMaxHeadDim = 128;  // WGSL_MAX_HEAD_DIM src/lib.rs:59-66
constexpr uint64_t kI32 = (uint64_t)std::numeric_limits<int32_t>::max();
// metadata part (block tables, lengths, positions, work list) of the allocation-free decode's
// scratch; the rest holds the queries' (cos, sin) rows and the split partials
constexpr size_t kNoAllocMetaBytes = (size_t)4 << 20;

bool mul_ov(uint64_t a, uint64_t b, uint64_t* out) {
    if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return true;
    *out = a * b;
    return false;
}

int elem_bytes(int dtype) { return dtype == FA_DTYPE_F32 ? 4 : 2; }

int check_dtype(int dtype) {
    if (dtype != FA_DTYPE_F32 && dtype != FA_DTYPE_F16 && dtype != FA_DTYPE_BF16)
        return fail(FA_ERR_UNSUPPORTED_DTYPE, "unsupported storage dtype %d", dtype);
    return FA_OK;
}

const char* dtype_name(int dtype) {
    return dtype == FA_DTYPE_F32 ? "f32" : dtype == FA_DTYPE_F16 ? "f16" : "bf16";
}

int resolve_scale(const fa_config* cfg, uint64_t head_dim, float* out) {
    if (head_dim == 0) return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
    float s = (cfg && cfg->has_softmax_scale) ? cfg->softmax_scale
                                              : 1.0f / std::sqrt((float)head_dim);
    if (!std::isfinite(s) || s <= 0.0f)
        return fail(FA_ERR_INVALID_SCALE, "softmax scale must be finite and positive, got %g",
                    (double)s);
    *out = s;
    return FA_OK;
}

// Head-dim support of the MFMA kernels: D <= 128; 16-bit storage needs D % 8 == 0 (16-byte
// row chunks); f32 storage accepts any D (RoPE additionally needs an even D).
int check_head_dim(uint64_t d, int dtype) {
    if (d > kMaxHeadDim)
        return fail(FA_ERR_UNSUPPORTED_HEAD_DIM, "head_dim %llu exceeds maximum %llu",
                    (unsigned long long)d, (unsigned long long)kMaxHeadDim);
    if (dtype != FA_DTYPE_F32 && d % 8 != 0)
        return fail(FA_ERR_UNSUPPORTED_HEAD_DIM,
                    "head_dim %llu is not a multiple of 8, required for %s storage",
                    (unsigned long long)d, dtype_name(dtype));
    return FA_OK;
}

int check_rotary(float theta, uint64_t offset, uint64_t head_dim, uint64_t len) {
    if (head_dim == 0 || head_dim % 2 != 0)
        return fail(FA_ERR_INVALID_ROTARY_HEAD_DIM,
                    "rotary attention head_dim must be non-zero and even, got %llu",
                    (unsigned long long)head_dim);
    if (!std::isfinite(theta) || theta <= 0.0f)
        return fail(FA_ERR_INVALID_ROTARY_THETA,
                    "rotary theta must be finite and positive, got %g", (double)theta);
    uint64_t last = len == 0 ? 0 : len - 1;
    if (offset > std::numeric_limits<uint64_t>::max() - last || offset + last > kI32)
        return fail(FA_ERR_POSITION_OVERFLOW,
                    "rotary position offset overflows the index space");
    return FA_OK;
}

int check_buffer(const char* name, const void* p, size_t have, uint64_t need) {
    if (!p) return fail(FA_ERR_NULL_ARGUMENT, "buffer %s is null", name);
    if ((uint64_t)have < need)
        return fail(FA_ERR_BUFFER_TOO_SMALL, "buffer %s contains %llu bytes, requires at least %llu",
                    name, (unsigned long long)have, (unsigned long long)need);
    return FA_OK;
}

uint64_t fnv1a64(const std::string& s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h;
}

// escape_component src/runtime_telemetry.rs:70-81: the record's delimiters inside a value
std::string escape_component(const char* v) {
    std::string out;
    for (const char* c = v; *c; ++c) {
        if (*c == '%') out += "%25";
        else if (*c == ';') out += "%3b";
        else if (*c == '=') out += "%3d";
        else out += *c;
    }
    return out;
}

std::string device_record(const char* name, const char* arch, int driver, int cus,
                          int clock_khz, uint64_t mem_bytes) {
    char tail[160];
    snprintf(tail, sizeof tail, ";driver=%d;cus=%d;clock_khz=%d;mem=%llu", driver, cus,
             clock_khz, (unsigned long long)mem_bytes);
    return "name=" + escape_component(name) + ";arch=" + escape_component(arch) + tail;
}

void copy_str(char* dst, size_t cap, const std::string& s) {
    size_t n = std::min(cap - 1, s.size());
    memcpy(dst, s.data(), n);
    dst[n] = 0;
}

}  // namespace

// ---------------------------------------------------------------------------- context
struct fa_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string name, arch;
    uint64_t fingerprint = 0;
    int prerotate_policy = -1;
    fa_telemetry last{};
    // (cos, sin) table cache, keyed by (theta, head_dim)
    float2* rope = nullptr;
    float rope_theta = 0.0f;
    uint64_t rope_dim = 0, rope_rows = 0;
    // growable scratch for the K pre-rotation pass
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // growable scratch for the backward's per-row (LSE log2 e, rowsum(dO * O))
    void* ws_delta = nullptr;
    size_t ws_delta_bytes = 0;
    // growable scratch for the backward's stored dS (16-bit storage; fa_ctx_set_backward_policy)
    void* ws_ds = nullptr;
    size_t ws_ds_bytes = 0;
    int backward_ds_policy = -1;
    // dK/dV kernel of the backward: -1 / 1 the assembly kernel where it applies, 0 HIP only
    int backward_kernel_policy = -1;
    // 16-bit RoPE prefill scores: 0 = rotated Q/K rounded to the storage type, 1 = split
    // high/residual operands (fa_ctx_set_prefill_precision)
    int prefill_precision = 0;
    // 16-bit contiguous prefill main loop: -1 (default) and 1 the assembly kernel where it
    // applies, 0 the HIP kernels (fa_ctx_set_prefill_kernel)
    int prefill_kernel_policy = -1;
    // the stream is being captured into a graph (fa_graph_capture_begin)
    bool capturing = false;
    // decode work layout: -1 automatic (head-grouped workgroups where they apply), 0 one-wave
    // workgroups (fa_ctx_set_decode_policy; read when a decode plan is prepared)
    int decode_grouped_policy = -1;
    // per-call metadata (variable-length prefill, batched append): one device buffer that each
    // call overwrites by a stream-ordered copy just before its launch
    int32_t* meta_dev = nullptr;
    size_t meta_dev_bytes = 0;
    // pinned host staging for stream-ordered uploads: a slot is reused once the event recorded
    // after its copy has completed, so no upload waits for the stream
    struct Staging {
        void* host = nullptr;
        size_t bytes = 0;
        hipEvent_t done = nullptr;
        bool busy = false;
    };
    std::vector<Staging> staging;
    // device buffers replaced by larger ones while work may still read them: freed at destroy
    std::vector<void*> retired;
    // per-call allocation accounting (telemetry)
    uint32_t call_allocs = 0;
    uint64_t call_alloc_bytes = 0;
    // per-kernel device timing (fa_ctx_set_kernel_timing)
    struct Span {
        int kernel_id;
        hipEvent_t begin, end;
    };
    bool timing = false;
    bool timing_paused = false;  // fa_ctx_pause_kernel_timing
    hipEvent_t open_begin = nullptr;
    std::vector<hipEvent_t> free_events;
    std::vector<Span> pending;
    // allocation-free decode: the device's static scratch (fa::noalloc_scratch, resolved when the
    // context is created), a host staging area for its metadata and the event that marks the
    // last copy out of that area
    void* na_scratch = nullptr;
    int32_t* na_host = nullptr;  // pinned, kNoAllocMetaBytes
    hipEvent_t na_copied = nullptr;
    bool na_pending = false;
    struct Timed {
        double total_ms = 0.0, min_ms = 0.0, max_ms = 0.0;
        uint64_t launches = 0;
    };
    std::vector<Timed> timed;  // indexed by kernel id
};

namespace {

int set_device(fa_ctx* ctx) {
    if (ctx->capturing) return FA_OK;  // made current when the capture began
    HIP_TRY(hipSetDevice(ctx->device));
    return FA_OK;
}

int refuse_in_capture(const fa_ctx* ctx, const char* what) {
    if (!ctx->capturing) return FA_OK;
    return fail(FA_ERR_GRAPH_CAPTURE,
                "%s while the stream is being captured; prepare plans and warm the context's "
                "caches before fa_graph_capture_begin", what);
}

void begin_call(fa_ctx* ctx) {
    ctx->call_allocs = 0;
    ctx->call_alloc_bytes = 0;
}

void fill_telemetry(fa_telemetry& t, const fa_ctx* ctx, int kernel_id, const char* name,
                    uint32_t qrows, uint32_t kvrows, const unsigned grid[3], unsigned block,
                    uint32_t dispatches, uint32_t splits, const char* fallback, uint32_t allocs,
                    uint64_t alloc_bytes) {
    memset(&t, 0, sizeof t);
    t.kernel_id = kernel_id;
    copy_str(t.kernel_name, sizeof t.kernel_name, name);
    t.query_rows = qrows;
    t.kv_rows = kvrows;
    t.workgroups[0] = grid[0];
    t.workgroups[1] = grid[1];
    t.workgroups[2] = grid[2];
    t.workgroup_size = block;
    t.dispatch_count = dispatches;
    t.temporary_allocation_count = allocs;
    t.temporary_allocation_bytes = alloc_bytes;
    t.splits = splits;
    if (fallback) {
        t.has_fallback_reason = 1;
        copy_str(t.fallback_reason, sizeof t.fallback_reason, fallback);
    }
    copy_str(t.device_name, sizeof t.device_name, ctx->name);
    copy_str(t.device_arch, sizeof t.device_arch, ctx->arch);
    t.device_fingerprint = ctx->fingerprint;
}

void record(fa_ctx* ctx, int kernel_id, const char* name, uint32_t qrows, uint32_t kvrows,
            const unsigned grid[3], unsigned block, uint32_t dispatches, uint32_t splits,
            const char* fallback) {
    fill_telemetry(ctx->last, ctx, kernel_id, name, qrows, kvrows, grid, block, dispatches,
                   splits, fallback, ctx->call_allocs, ctx->call_alloc_bytes);
}

// Timing marks: begin_span records an event before a dispatch, end_span one after it and
// files the pair under `kernel_id`. Both are no-ops while timing is off; an event failure
// drops that one measurement rather than failing the call.
hipEvent_t take_event(fa_ctx* ctx) {
    if (!ctx->free_events.empty()) {
        hipEvent_t e = ctx->free_events.back();
        ctx->free_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    return hipEventCreate(&e) == hipSuccess ? e : nullptr;
}

void begin_span(fa_ctx* ctx) {
    if (!ctx->timing || ctx->timing_paused || ctx->capturing) return;
    hipEvent_t e = take_event(ctx);
    if (e && hipEventRecord(e, ctx->stream) != hipSuccess) {
        ctx->free_events.push_back(e);
        e = nullptr;
    }
    ctx->open_begin = e;
}

// The span of a dispatch that records its own start and stop events (hipExtModuleLaunchKernel):
// false while timing is off or without events, and then the caller brackets it with
// begin_span / end_span.
bool dispatch_events(fa_ctx* ctx, hipEvent_t* start, hipEvent_t* stop) {
    *start = *stop = nullptr;
    if (!ctx->timing || ctx->timing_paused || ctx->capturing) return false;
    *start = take_event(ctx);
    *stop = take_event(ctx);
    if (*start && *stop) return true;
    if (*start) ctx->free_events.push_back(*start);
    if (*stop) ctx->free_events.push_back(*stop);
    *start = *stop = nullptr;
    return false;
}

void end_span(fa_ctx* ctx, int kernel_id) {
    if (!ctx->timing || ctx->timing_paused || ctx->capturing || !ctx->open_begin) return;
    hipEvent_t e = take_event(ctx);
    if (!e || hipEventRecord(e, ctx->stream) != hipSuccess) {
        ctx->free_events.push_back(ctx->open_begin);
        if (e) ctx->free_events.push_back(e);
    } else {
        ctx->pending.push_back({kernel_id, ctx->open_begin, e});
    }
    ctx->open_begin = nullptr;
}

// Folds completed spans into the per-kernel totals (waits for the stream first).
int resolve_spans(fa_ctx* ctx) {
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    for (const auto& s : ctx->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, s.begin, s.end) == hipSuccess && s.kernel_id >= 0) {
            if ((size_t)s.kernel_id >= ctx->timed.size()) ctx->timed.resize(s.kernel_id + 1);
            fa_ctx::Timed& t = ctx->timed[s.kernel_id];
            t.min_ms = t.launches ? std::min(t.min_ms, (double)ms) : ms;
            t.max_ms = t.launches ? std::max(t.max_ms, (double)ms) : ms;
            t.total_ms += ms;
            t.launches += 1;
        }
        ctx->free_events.push_back(s.begin);
        ctx->free_events.push_back(s.end);
    }
    ctx->pending.clear();
    return FA_OK;
}

int dev_alloc(fa_ctx* ctx, void** p, size_t bytes) {
    if (int rc = refuse_in_capture(ctx, "device allocation")) return rc;
    HIP_TRY(hipMalloc(p, bytes ? bytes : 16));
    ctx->call_allocs += 1;
    ctx->call_alloc_bytes += bytes;
    return FA_OK;
}

// inv_freq[p] = theta^(-2p/D) in f32 with the host powf, as rotated_pair computes it
fa::RopeFreqs rope_freqs(float theta, uint64_t head_dim) {
    fa::RopeFreqs f{};
    for (uint64_t p = 0; p < head_dim / 2; ++p) {
        float exponent = -2.0f * (float)p / (float)head_dim;
        f.inv_freq[p] = powf(theta, exponent);
    }
    return f;
}

// Builds a (cos, sin) table of `rows` positions into `table` on the context's stream.
int build_rope_table(fa_ctx* ctx, float2* table, float theta, uint64_t head_dim, uint64_t rows) {
    begin_span(ctx);
    fa::launch_rope_table(table, rope_freqs(theta, head_dim), (int)rows, (int)(head_dim / 2),
                          ctx->stream);
    end_span(ctx, FA_KERNEL_ROPE_TABLE);
    HIP_TRY(hipGetLastError());
    return FA_OK;
}

// (cos, sin) table covering positions [0, rows) for (theta, head_dim), cached by the context.
// A larger table replaces the cached one without waiting for the stream (the old one is
// retired).
int ensure_rope(fa_ctx* ctx, float theta, uint64_t head_dim, uint64_t rows, const float2** out) {
    if (ctx->rope && ctx->rope_theta == theta && ctx->rope_dim == head_dim &&
        ctx->rope_rows >= rows) {
        *out = ctx->rope;
        return FA_OK;
    }
    uint64_t cap = std::max<uint64_t>(rows, 4096);
    if (ctx->rope_theta == theta && ctx->rope_dim == head_dim)
        cap = std::max<uint64_t>(cap, ctx->rope_rows * 2);
    float2* fresh = nullptr;
    if (int rc = dev_alloc(ctx, (void**)&fresh, cap * (head_dim / 2) * sizeof(float2))) return rc;
    if (ctx->rope) ctx->retired.push_back(ctx->rope);
    ctx->rope = fresh;
    ctx->rope_theta = theta;
    ctx->rope_dim = head_dim;
    ctx->rope_rows = cap;
    if (int rc = build_rope_table(ctx, fresh, theta, head_dim, cap)) return rc;
    *out = ctx->rope;
    return FA_OK;
}

// Grows a context-owned buffer without waiting for the stream: work already enqueued keeps
// reading the old buffer, which is retired (freed when the context is destroyed).
int grow(fa_ctx* ctx, void** buf, size_t* cap, size_t bytes, void** out) {
    if (*cap < bytes) {
        void* fresh = nullptr;
        if (int rc = dev_alloc(ctx, &fresh, bytes)) return rc;
        if (*buf) ctx->retired.push_back(*buf);
        *buf = fresh;
        *cap = bytes;
    }
    *out = *buf;
    return FA_OK;
}

// Stream-ordered host -> device copy of `bytes` from `src` through a pinned staging slot. The
// host never waits: a slot whose previous copy has not completed is skipped and, when none is
// free, a new slot is allocated.
int stage_upload(fa_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!bytes) return FA_OK;
    if (int rc = refuse_in_capture(ctx, "host upload")) return rc;
    fa_ctx::Staging* slot = nullptr;
    for (auto& st : ctx->staging) {
        if (st.busy && hipEventQuery(st.done) == hipSuccess) st.busy = false;
        if (!st.busy && st.bytes >= bytes && (!slot || st.bytes < slot->bytes)) slot = &st;
    }
    if (!slot) {
        fa_ctx::Staging st;
        st.bytes = std::max<size_t>(bytes, 4096);
        HIP_TRY(hipHostMalloc(&st.host, st.bytes, hipHostMallocDefault));
        if (hipEventCreateWithFlags(&st.done, hipEventDisableTiming) != hipSuccess) {
            (void)hipHostFree(st.host);
            return fail(FA_ERR_HIP, "hipEventCreateWithFlags failed");
        }
        ctx->staging.push_back(st);
        slot = &ctx->staging.back();
    }
    memcpy(slot->host, src, bytes);
    HIP_TRY(hipMemcpyAsync(dst, slot->host, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipEventRecord(slot->done, ctx->stream));
    slot->busy = true;
    return FA_OK;
}

int ensure_ws(fa_ctx* ctx, size_t bytes, void** out) {
    return grow(ctx, &ctx->ws, &ctx->ws_bytes, bytes, out);
}

// Stream-ordered upload of `n` int32 values to the context's metadata buffer: a later launch on
// the stream reads them, an earlier one has finished with the previous contents (same stream).
int upload_meta(fa_ctx* ctx, const int32_t* vals, size_t n, const int32_t** dev) {
    const size_t bytes = n * sizeof(int32_t);
    void* d = nullptr;
    if (int rc = grow(ctx, (void**)&ctx->meta_dev, &ctx->meta_dev_bytes, bytes, &d)) return rc;
    if (int rc = stage_upload(ctx, d, vals, bytes)) return rc;
    *dev = (const int32_t*)d;
    return FA_OK;
}

}  // namespace

extern "C" {

int fa_abi_version(void) { return FA_ABI_VERSION; }

const char* fa_last_error_message(void) { return g_error.c_str(); }

const char* fa_status_string(int s) {
    switch (s) {
        case FA_OK: return "ok";
        case FA_ERR_ZERO_DIMENSION: return "ZeroDimension";
        case FA_ERR_SHAPE_OVERFLOW: return "ShapeOverflow";
        case FA_ERR_INVALID_HEAD_GROUPING: return "InvalidHeadGrouping";
        case FA_ERR_INVALID_ROTARY_HEAD_DIM: return "InvalidRotaryHeadDim";
        case FA_ERR_INVALID_ROTARY_THETA: return "InvalidRotaryTheta";
        case FA_ERR_POSITION_OVERFLOW: return "PositionOverflow";
        case FA_ERR_LENGTH_MISMATCH: return "LengthMismatch";
        case FA_ERR_INVALID_SCALE: return "InvalidScale";
        case FA_ERR_NON_FINITE_INPUT: return "NonFiniteInput";
        case FA_ERR_UNAVAILABLE: return "Unavailable";
        case FA_ERR_UNSUPPORTED_HEAD_DIM: return "UnsupportedHeadDim";
        case FA_ERR_FOREIGN_BUFFER: return "ForeignBuffer";
        case FA_ERR_INDEX_SPACE_EXCEEDED: return "IndexSpaceExceeded";
        case FA_ERR_DISPATCH_LIMIT: return "DispatchLimit";
        case FA_ERR_BUFFER_TOO_SMALL: return "BufferTooSmall";
        case FA_ERR_EMPTY_TABLE: return "EmptyTable";
        case FA_ERR_TOO_MANY_MAPPED_PAGES: return "TooManyMappedPages";
        case FA_ERR_CAUSAL_VISIBILITY_MISMATCH: return "CausalVisibilityMismatch";
        case FA_ERR_ZERO_QUERY_CHUNK_SIZE: return "ZeroQueryChunkSize";
        case FA_ERR_UNSUPPORTED_DTYPE: return "UnsupportedDtype";
        case FA_ERR_INVALID_PAGE: return "InvalidPage";
        case FA_ERR_EMPTY_CACHE: return "EmptyCache";
        case FA_ERR_INVALID_CACHE_LENGTH: return "InvalidCacheLength";
        case FA_ERR_PAGED_ZERO_DIMENSION: return "PagedZeroDimension";
        case FA_ERR_CAPACITY_OVERFLOW: return "CapacityOverflow";
        case FA_ERR_CAPACITY_EXCEEDED: return "CapacityExceeded";
        case FA_ERR_GENERATION_OVERFLOW: return "GenerationOverflow";
        case FA_ERR_NULL_ARGUMENT: return "NullArgument";
        case FA_ERR_HIP: return "Hip";
        case FA_ERR_SCRATCH_EXCEEDED: return "ScratchExceeded";
        default: return "Unknown";
    }
}

int fa_resolved_scale(const fa_config* config, uint64_t head_dim, float* out) {
    if (!out) return fail(FA_ERR_NULL_ARGUMENT, "output pointer is null");
    int rc = resolve_scale(config, head_dim, out);
    return rc ? rc : ok();
}

int fa_packed_layout_for(uint64_t output_elements, uint64_t lse_elements, int dtype,
                         fa_packed_layout* out) {
    if (!out) return fail(FA_ERR_NULL_ARGUMENT, "output pointer is null");
    if (int rc = check_dtype(dtype)) return rc;
    uint64_t ob, lb;
    if (mul_ov(output_elements, (uint64_t)elem_bytes(dtype), &ob) || mul_ov(lse_elements, 4, &lb))
        return fail(FA_ERR_SHAPE_OVERFLOW, "attention shape overflows the address space");
    out->output_elements = output_elements;
    out->lse_elements = lse_elements;
    out->output_bytes = ob;
    out->lse_byte_offset = (ob + 3) & ~3ull;
    out->combined_bytes = out->lse_byte_offset + lb;
    return ok();
}

int fa_ctx_create(int device, fa_ctx** out) {
    if (!out) return fail(FA_ERR_NULL_ARGUMENT, "output pointer is null");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        return fail(FA_ERR_UNAVAILABLE, "no HIP device is available");
    if (device < 0 || device >= count)
        return fail(FA_ERR_UNAVAILABLE, "HIP device %d does not exist (%d present)", device, count);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    std::string arch = prop.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
        return fail(FA_ERR_UNAVAILABLE, "device %d is %s; this backend is built for gfx950 only",
                    device, arch.c_str());
    HIP_TRY(hipSetDevice(device));
    fa_ctx* ctx = new fa_ctx();
    ctx->device = device;
    // some drivers report no marketing name: name the part by its architecture instead
    ctx->name = prop.name[0] ? std::string(prop.name) : "AMD " + arch.substr(0, arch.find(':'));
    ctx->arch = arch;
    int drv = 0;
    (void)hipDriverGetVersion(&drv);
    ctx->fingerprint = fnv1a64(device_record(ctx->name.c_str(), arch.c_str(), drv,
                                             prop.multiProcessorCount, prop.clockRate,
                                             (uint64_t)prop.totalGlobalMem));
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return fail(FA_ERR_HIP, "hipStreamCreate failed");
    }
    // set-up of the allocation-free decode (device current): the scratch address of this
    // device and the host staging area; a failure here surfaces at that entry point
    if (fa::noalloc_scratch(device, &ctx->na_scratch) != hipSuccess) ctx->na_scratch = nullptr;
    // the assembly prefill's code object (a load failure leaves the HIP kernels in use, which
    // the telemetry's kernel name shows)
    (void)fa::prefill_a64_load(device);
    (void)fa::bwd_a64_load(device);
    if (hipEventCreateWithFlags(&ctx->na_copied, hipEventDisableTiming) != hipSuccess)
        ctx->na_copied = nullptr;
    if (hipHostMalloc((void**)&ctx->na_host, kNoAllocMetaBytes, hipHostMallocDefault) !=
        hipSuccess)
        ctx->na_host = nullptr;
    *out = ctx;
    return ok();
}

int fa_ctx_destroy(fa_ctx* ctx) {
    if (!ctx) return ok();
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->rope) (void)hipFree(ctx->rope);
    for (void* r : ctx->retired) (void)hipFree(r);
    for (auto& st : ctx->staging) {
        (void)hipHostFree(st.host);
        (void)hipEventDestroy(st.done);
    }
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->ws_delta) (void)hipFree(ctx->ws_delta);
    if (ctx->ws_ds) (void)hipFree(ctx->ws_ds);
    if (ctx->meta_dev) (void)hipFree(ctx->meta_dev);
    for (const auto& s : ctx->pending) {
        (void)hipEventDestroy(s.begin);
        (void)hipEventDestroy(s.end);
    }
    if (ctx->open_begin) (void)hipEventDestroy(ctx->open_begin);
    if (ctx->na_copied) (void)hipEventDestroy(ctx->na_copied);
    if (ctx->na_host) (void)hipHostFree(ctx->na_host);
    for (hipEvent_t e : ctx->free_events) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return ok();
}

void* fa_ctx_stream(fa_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int fa_ctx_synchronize(fa_ctx* ctx) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    if (int rc = refuse_in_capture(ctx, "stream synchronisation")) return rc;
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return ok();
}

int fa_ctx_device_name(fa_ctx* ctx, char* buf, size_t len) {
    if (!ctx || !buf || !len) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    copy_str(buf, len, ctx->name + " (" + ctx->arch + ")");
    return ok();
}

int fa_device_record(const char* name, const char* arch, int32_t driver, int32_t cus,
                     int32_t clock_khz, uint64_t mem_bytes, char* out, size_t cap,
                     uint64_t* fingerprint) {
    if (!name || !arch || !fingerprint) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    const std::string rec = device_record(name, arch, driver, cus, clock_khz, mem_bytes);
    if (out && cap) copy_str(out, cap, rec);
    *fingerprint = fnv1a64(rec);
    return ok();
}

int fa_ctx_set_kernel_timing(fa_ctx* ctx, int32_t enable) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    if (int rc = set_device(ctx)) return rc;
    if (int rc = resolve_spans(ctx)) return rc;
    ctx->timed.clear();
    ctx->timing = enable != 0;
    ctx->timing_paused = false;
    return ok();
}

int fa_ctx_pause_kernel_timing(fa_ctx* ctx, int32_t paused) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    ctx->timing_paused = paused != 0;
    return ok();
}

int fa_ctx_kernel_timing(fa_ctx* ctx, int32_t kernel_id, double* total_ms, uint64_t* launches) {
    if (!ctx || !total_ms || !launches) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = set_device(ctx)) return rc;
    if (int rc = resolve_spans(ctx)) return rc;
    *total_ms = 0.0;
    *launches = 0;
    if (kernel_id >= 0 && (size_t)kernel_id < ctx->timed.size()) {
        *total_ms = ctx->timed[kernel_id].total_ms;
        *launches = ctx->timed[kernel_id].launches;
    }
    return ok();
}

int fa_ctx_kernel_timing_range(fa_ctx* ctx, int32_t kernel_id, double* min_ms, double* max_ms) {
    if (!ctx || !min_ms || !max_ms) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = set_device(ctx)) return rc;
    if (int rc = resolve_spans(ctx)) return rc;
    *min_ms = 0.0;
    *max_ms = 0.0;
    if (kernel_id >= 0 && (size_t)kernel_id < ctx->timed.size()) {
        *min_ms = ctx->timed[kernel_id].min_ms;
        *max_ms = ctx->timed[kernel_id].max_ms;
    }
    return ok();
}

int fa_ctx_set_decode_policy(fa_ctx* ctx, int32_t grouped) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    ctx->decode_grouped_policy = grouped < 0 ? -1 : (grouped ? 1 : 0);
    return ok();
}

int fa_ctx_set_backward_policy(fa_ctx* ctx, int32_t store_ds) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    ctx->backward_ds_policy = store_ds < 0 ? -1 : (store_ds ? 1 : 0);
    return ok();
}

int fa_ctx_set_prefill_precision(fa_ctx* ctx, int32_t mode) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    if (mode != 0 && mode != 1)
        return fail(FA_ERR_UNAVAILABLE, "prefill precision mode %d is not one of 0, 1", (int)mode);
    ctx->prefill_precision = mode;
    return ok();
}

int fa_ctx_set_prefill_kernel(fa_ctx* ctx, int32_t assembly) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    ctx->prefill_kernel_policy = assembly < 0 ? -1 : (assembly ? 1 : 0);
    return ok();
}

int fa_ctx_set_backward_kernel(fa_ctx* ctx, int32_t assembly) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    ctx->backward_kernel_policy = assembly < 0 ? -1 : (assembly ? 1 : 0);
    return ok();
}

int fa_ctx_set_prefill_policy(fa_ctx* ctx, int32_t prerotate_k) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    ctx->prerotate_policy = prerotate_k < 0 ? -1 : (prerotate_k ? 1 : 0);
    return ok();
}

// ---------------------------------------------------------------------------- buffers
int fa_buf_alloc(fa_ctx* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = refuse_in_capture(ctx, "buffer allocation or copy")) return rc;
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipMalloc(out, bytes ? bytes : 16));
    return ok();
}

int fa_buf_free(fa_ctx* ctx, void* ptr) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    if (int rc = refuse_in_capture(ctx, "buffer allocation or copy")) return rc;
    if (!ptr) return ok();
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    HIP_TRY(hipFree(ptr));
    return ok();
}

int fa_buf_upload(fa_ctx* ctx, void* dst, const void* host, size_t bytes) {
    if (!ctx || !dst || (!host && bytes)) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = refuse_in_capture(ctx, "buffer allocation or copy")) return rc;
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return ok();
}

int fa_buf_download(fa_ctx* ctx, void* host, const void* src, size_t bytes) {
    if (!ctx || !src || (!host && bytes)) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = refuse_in_capture(ctx, "buffer allocation or copy")) return rc;
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipMemcpyAsync(host, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return ok();
}

int fa_buf_fill_u32(fa_ctx* ctx, void* dst, uint32_t value, size_t count) {
    if (!ctx || !dst) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    // a memset node must not enter a graph: its replays have given wrong results on this part
    if (int rc = refuse_in_capture(ctx, "buffer fill")) return rc;
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipMemsetD32Async((hipDeviceptr_t)dst, (int)value, count, ctx->stream));
    return ok();
}

// ------------------------------------------------------------------------------ graphs
struct fa_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int device = 0;
};

int fa_graph_capture_begin(fa_ctx* ctx) {
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    if (ctx->capturing) return fail(FA_ERR_GRAPH_CAPTURE, "the stream is already being captured");
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    return ok();
}

int fa_graph_capture_end(fa_ctx* ctx, fa_graph** out) {
    if (!ctx || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    if (!ctx->capturing) return fail(FA_ERR_GRAPH_CAPTURE, "the stream is not being captured");
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamEndCapture(ctx->stream, &g));
    hipGraphExec_t e = nullptr;
    const hipError_t err = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    if (err != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(FA_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(err));
    }
    fa_graph* r = new fa_graph();
    r->graph = g;
    r->exec = e;
    r->device = ctx->device;
    *out = r;
    return ok();
}

int fa_graph_launch(fa_ctx* ctx, const fa_graph* graph) {
    if (!ctx || !graph) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (graph->device != ctx->device)
        return fail(FA_ERR_FOREIGN_BUFFER, "graph was captured on device %d, context is on %d",
                    graph->device, ctx->device);
    if (int rc = refuse_in_capture(ctx, "graph launch")) return rc;
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipGraphLaunch(graph->exec, ctx->stream));
    return ok();
}

int fa_graph_destroy(fa_graph* graph) {
    if (!graph) return ok();
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
    return ok();
}

int fa_last_telemetry(fa_ctx* ctx, fa_telemetry* out) {
    if (!ctx || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    *out = ctx->last;
    return ok();
}

}  // extern "C"

// ---------------------------------------------------------------------------- prefill core
namespace {

bool want_prerotate(const fa_ctx* ctx, uint64_t head_dim) {
    if (head_dim % 8 != 0) return false;  // the pre-pass moves 8-element chunks
    if (ctx->prerotate_policy >= 0) return ctx->prerotate_policy == 1;
    return true;  // default: rotate K once, then stream pre-rotated K tiles
}

int prefill_kernel_id(int dtype, bool prerot) {
    if (dtype == FA_DTYPE_BF16) return prerot ? FA_KERNEL_PREFILL_MFMA_BF16_PREROT : FA_KERNEL_PREFILL_MFMA_BF16;
    if (dtype == FA_DTYPE_F16) return prerot ? FA_KERNEL_PREFILL_MFMA_F16_PREROT : FA_KERNEL_PREFILL_MFMA_F16;
    return prerot ? FA_KERNEL_PREFILL_MFMA_F32_PREROT : FA_KERNEL_PREFILL_MFMA_F32;
}

const char* kernel_name(int id) {
    switch (id) {
        case FA_KERNEL_PREFILL_MFMA_BF16: return "prefill_mfma16<bf16> (K rotated on load)";
        case FA_KERNEL_PREFILL_MFMA_F16: return "prefill_mfma16<f16> (K rotated on load)";
        case FA_KERNEL_PREFILL_MFMA_F32: return "prefill_mfma_f32";
        case FA_KERNEL_PREFILL_MFMA_BF16_PREROT: return "rotate_rows + prefill_mfma16<bf16>";
        case FA_KERNEL_PREFILL_MFMA_F16_PREROT: return "rotate_rows + prefill_mfma16<f16>";
        case FA_KERNEL_PREFILL_MFMA_F32_PREROT: return "rotate_rows + prefill_mfma_f32";
        case FA_KERNEL_DECODE_PAGED_SPLITK: return "decode_splitk + decode_combine";
        case FA_KERNEL_DECODE_PAGED_MFMA: return "decode_mfma + decode_combine";
        default: return "none";
    }
}

// Closes the split kernel's timing span and opens the combine's, between the two launches
// (own: the split kernel recorded its span's events in its dispatch, which are filed here).
struct DecodeMarks {
    fa_ctx* ctx;
    const bool* mfma;
    bool own = false;
    hipEvent_t start = nullptr, stop = nullptr;
    static void between(void* user) {
        auto* m = static_cast<DecodeMarks*>(user);
        const int kid = *m->mfma ? FA_KERNEL_DECODE_PAGED_MFMA : FA_KERNEL_DECODE_PAGED_SPLITK;
        if (m->own)
            m->ctx->pending.push_back({kid, m->start, m->stop});
        else
            end_span(m->ctx, kid);
        begin_span(m->ctx);
    }
};

// Common launch of the prefill kernel. `k_layout_rows`/`k_period`/`k_heads` describe how to
// pre-rotate contiguous K (rows of k_heads*D elements, row r at position kv_rope_offset +
// r % k_period) when the pre-rotation variant is selected.
struct PrefillJob {
    fa::PrefillArgs a;
    Dtype dt;
    int dtype;
    bool paged = false;
    bool rope = false;
    float theta = 0.0f;
    uint64_t max_pos = 0;  // highest RoPE position used + 1
    uint64_t kv_bytes = 0;
    uint64_t k_rows = 0, k_heads = 0, k_period = 0;
};

// The resolved form of a prefill job: variant decisions and the device memory the launch uses
// (the context's caches for a one-shot call, memory owned by a prepared forward otherwise).
struct PrefillRun {
    PrefillJob j;
    bool prerot = false;
    bool prec64 = false;      // precise scores in the assembly kernel (K and its residual)
    float2* table = nullptr;  // RoPE (cos, sin) rows [0, max_pos)
    void* ws = nullptr;       // rotated K (prerot)
};

// Decides the variant and gathers the memory. own == false: the context's growable caches;
// own == true: fresh allocations that the caller (a prepared forward) keeps and frees.
// Variant decisions of a prefill job under the context's policies (no device work).
struct PrefillChoice {
    bool prerot = false;  // K rotated once by the pre-pass
    bool split_qk = false;  // precise 16-bit scores: K rotated on load, split Q/K
    bool prec64 = false;  // precise 16-bit scores in the assembly kernel: K and its residual
                          // from the pre-pass (prerot), Q split in the kernel
};

PrefillChoice choose_prefill(const fa_ctx* ctx, const PrefillJob& j) {
    PrefillChoice c;
    if (j.rope) {
        c.prerot = j.a.rope_k && !j.paged && want_prerotate(ctx, (uint64_t)j.a.head_dim);
        if (ctx->prefill_precision == 1 && j.a.rope_k && !j.paged && j.dtype != FA_DTYPE_F32) {
            // the assembly kernel where it takes the launch (the arguments it would receive:
            // K rotated by the pre-pass, the residual beside it), else the HIP split kernel
            fa::PrefillArgs t = j.a;
            t.rope_k = 0;
            t.a64 = ctx->prefill_kernel_policy != 0;
            t.rope_rows = (int)j.max_pos;
            t.rope_table = (const float2*)(uintptr_t)16;
            t.k_lo = (const void*)(uintptr_t)16;
            if (j.dtype == FA_DTYPE_BF16 && j.a.head_dim % 8 == 0 &&
                fa::prefill_a64_eligible(j.dt, false, t)) {
                c.prerot = true;
                c.prec64 = true;
            } else {
                c.prerot = false;
                c.split_qk = true;
            }
        }
    }
    return c;
}

// Bytes of the rotated-K workspace: the rotation, and for the precise assembly kernel its
// residual right after it.
uint64_t ws_bytes_for(const PrefillJob& j, const PrefillChoice& c) {
    return c.prec64 ? 2 * j.kv_bytes : j.kv_bytes;
}

// Device allocations a one-shot call of `j` would make through the context's growable caches
// (RoPE table, rotated-K workspace), given what they hold now.
void predict_prefill_allocs(const fa_ctx* ctx, const PrefillJob& j, const PrefillChoice& c,
                            uint32_t* count, uint64_t* bytes) {
    *count = 0;
    *bytes = 0;
    const uint64_t hd = (uint64_t)j.a.head_dim;
    if (j.rope && !(ctx->rope && ctx->rope_theta == j.theta && ctx->rope_dim == hd &&
                    ctx->rope_rows >= j.max_pos)) {
        uint64_t cap = std::max<uint64_t>(j.max_pos, 4096);
        if (ctx->rope_theta == j.theta && ctx->rope_dim == hd)
            cap = std::max<uint64_t>(cap, ctx->rope_rows * 2);
        ++*count;
        *bytes += cap * (hd / 2) * sizeof(float2);
    }
    if (c.prerot && ctx->ws_bytes < ws_bytes_for(j, c)) {
        ++*count;
        *bytes += ws_bytes_for(j, c);
    }
}

int resolve_prefill(fa_ctx* ctx, PrefillJob& j, bool own, PrefillRun* r) {
    // 16-bit contiguous K/V are read through 32-bit buffer offsets within one (batch, kv-head)
    // slice: kv_len rows of k_ss elements must stay below 2 GiB.
    if (!j.paged && j.dtype != FA_DTYPE_F32 &&
        (uint64_t)j.a.kv_len * (uint64_t)j.a.k_ss * 2u > (uint64_t)INT32_MAX)
        return fail(FA_ERR_INDEX_SPACE_EXCEEDED,
                    "one K/V slice spans %llu bytes; the 16-bit kernels address at most 2 GiB",
                    (unsigned long long)((uint64_t)j.a.kv_len * (uint64_t)j.a.k_ss * 2u));
    r->j = j;
    bool prerot = false;
    if (j.rope) {
        if (own) {
            if (int rc = dev_alloc(ctx, (void**)&r->table,
                                   j.max_pos * ((uint64_t)j.a.head_dim / 2) * sizeof(float2)))
                return rc;
            if (int rc = build_rope_table(ctx, r->table, j.theta, (uint64_t)j.a.head_dim,
                                          j.max_pos))
                return rc;
        } else {
            const float2* t = nullptr;
            if (int rc = ensure_rope(ctx, j.theta, (uint64_t)j.a.head_dim, j.max_pos, &t))
                return rc;
            r->table = const_cast<float2*>(t);
        }
        r->j.a.rope_table = r->table;
        const PrefillChoice c = choose_prefill(ctx, j);
        prerot = c.prerot;
        r->prec64 = c.prec64;
        // precise scores: K rotated in the kernel, which keeps its 16-bit residual
        if (c.split_qk) r->j.a.split_qk = 1;
        r->j.a.rope_rows = (int)j.max_pos;
    }
    r->j.a.a64 = ctx->prefill_kernel_policy != 0;
    r->prerot = prerot;
    if (prerot) {
        const uint64_t wsb = r->prec64 ? 2 * j.kv_bytes : j.kv_bytes;
        if (own) {
            if (int rc = dev_alloc(ctx, &r->ws, wsb)) return rc;
        } else if (int rc = ensure_ws(ctx, wsb, &r->ws)) {
            return rc;
        }
    }
    return FA_OK;
}

// Telemetry of a prefill whose kernel arguments are `a` (after the pre-passes' substitutions):
// kernel id and name, geometry, dispatch count, allocations and the fallback reason.
void describe_prefill(const fa_ctx* ctx, const PrefillJob& j, const fa::PrefillArgs& a,
                      bool prerot, uint32_t dispatches, uint32_t allocs,
                      uint64_t alloc_bytes, fa_telemetry* out) {
    // K read already rotated (pre-pass, or a paged cache that stores K rotated on append)
    const int kid = prefill_kernel_id(j.dtype, prerot || (j.paged && j.rope));
    unsigned grid[3], block = 0, rows = 0;
    fa::prefill_geometry(j.dt, j.paged, a, grid, &block, &rows);
    const char* fb = nullptr;

    if (j.rope && a.rope_k && !prerot && !j.paged && a.head_dim % 8 != 0)
        fb = "K pre-rotation pass needs head_dim % 8 == 0; K rotated on load";
    const char* dt = j.dtype == FA_DTYPE_BF16 ? "bf16" : j.dtype == FA_DTYPE_F16 ? "f16" : "f32";
    const bool a64 = fa::prefill_a64_eligible(j.dt, j.paged, a);
    const char* base =
        j.dtype == FA_DTYPE_F32 ? "prefill_mfma_f32" : (a64 ? "prefill_a64" : "prefill_mfma16");
    char name[64];
    if (prerot && a.k_lo && a64)
        snprintf(name, sizeof name, "rotate_rows + %s<%s> (split Q/K scores)", base, dt);
    else if (prerot)
        snprintf(name, sizeof name, "rotate_rows + %s<%s>", base, dt);
    else if (j.paged)
        snprintf(name, sizeof name, "%s<%s> (paged%s)", base, dt, j.rope ? ", K stored rotated" : "");
    else if (a.split_qk)
        snprintf(name, sizeof name, "%s<%s> (K rotated on load, split Q/K scores)", base, dt);
    else if (a.rope_k)
        snprintf(name, sizeof name, "%s<%s> (K rotated on load)", base, dt);
    else
        snprintf(name, sizeof name, "%s<%s>", base, dt);
    fill_telemetry(*out, ctx, kid, name, rows, 64, grid, block, dispatches, 1, fb, allocs,
                   alloc_bytes);
}

// Enqueues the resolved prefill on the context's stream: the optional K pre-rotation pass, then
// the prefill kernel. No allocation, copy or wait.
int enqueue_prefill(fa_ctx* ctx, const PrefillRun& r) {
    fa::PrefillArgs a = r.j.a;
    const PrefillJob& j = r.j;
    uint32_t dispatches = 0;
    if (r.prerot) {
        begin_span(ctx);
        if (r.prec64)
            fa::launch_rotate_rows_split(a.k, r.ws, (uint8_t*)r.ws + j.kv_bytes, (int)j.k_rows,
                                         (int)j.k_heads, a.head_dim, (int64_t)j.k_period,
                                         r.table, a.kv_rope_offset, ctx->stream);
        else
            fa::launch_rotate_rows(j.dt, a.k, r.ws, (int)j.k_rows, (int)j.k_heads, a.head_dim,
                                   (int64_t)j.k_period, r.table, a.kv_rope_offset, ctx->stream);
        end_span(ctx, FA_KERNEL_ROPE_ROTATE);
        HIP_TRY(hipGetLastError());
        a.k = r.ws;
        a.rope_k = 0;
        if (r.prec64) a.k_lo = (const uint8_t*)r.ws + j.kv_bytes;
        dispatches++;
    }
    unsigned grid[3], block = 0;
    // K read already rotated (pre-pass, or a paged cache that stores K rotated on append)
    const int kid = prefill_kernel_id(j.dtype, r.prerot || (j.paged && j.rope));
    // the assembly and the f32 kernel (one dispatch each) record their span's events as part of
    // their dispatch
    const bool own = (j.dtype == FA_DTYPE_F32 || fa::prefill_a64_eligible(j.dt, j.paged, a)) &&
                     dispatch_events(ctx, &a.ev_start, &a.ev_stop);
    if (!own) begin_span(ctx);
    fa::launch_prefill(j.dt, j.paged, a, ctx->stream, grid, &block);
    if (own)
        ctx->pending.push_back({kid, a.ev_start, a.ev_stop});
    else
        end_span(ctx, kid);
    HIP_TRY(hipGetLastError());
    dispatches++;
    describe_prefill(ctx, j, a, r.prerot, dispatches, ctx->call_allocs,
                     ctx->call_alloc_bytes, &ctx->last);
    return FA_OK;
}

int run_prefill(fa_ctx* ctx, PrefillJob& j) {
    PrefillRun r;
    if (int rc = resolve_prefill(ctx, j, false, &r)) return rc;
    return enqueue_prefill(ctx, r);
}

int validate_grouped(uint64_t b, uint64_t hq, uint64_t hkv, uint64_t s, uint64_t d) {
    if (!b || !hq || !hkv || !s || !d)
        return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
    if (hq % hkv)
        return fail(FA_ERR_INVALID_HEAD_GROUPING,
                    "q_heads (%llu) must be exactly divisible by kv_heads (%llu)",
                    (unsigned long long)hq, (unsigned long long)hkv);
    uint64_t t;
    // the byte sizes too (up to 4 bytes per element) must fit, or a buffer check would wrap
    if (mul_ov(b, hq, &t) || mul_ov(t, s, &t) || mul_ov(t, d, &t) || mul_ov(t, 4, &t))
        return fail(FA_ERR_SHAPE_OVERFLOW, "attention shape overflows the address space");
    if (s > kI32 / std::max<uint64_t>(1, hq / hkv) || b * hkv > kI32)
        return fail(FA_ERR_INDEX_SPACE_EXCEEDED, "attention exceeds the i32 index space at %llu rows",
                    (unsigned long long)s);
    return FA_OK;
}

}  // namespace

extern "C" {

}  // extern "C"

namespace {

// Validation and kernel arguments of the contiguous grouped (optionally RoPE) forward, shared by
// the one-shot call and the prepared forward.
int build_gqa_job(fa_ctx* ctx, const void* q, size_t q_bytes, const void* k, const void* v,
                  size_t kv_bytes, void* out_lse, size_t out_bytes, const fa_grouped_shape* sh,
                  const fa_config* cfg, const fa_rotary* rot, int dtype, PrefillJob& j,
                  fa_packed_layout* layout, bool check_buffers = true) {
    if (!sh) return fail(FA_ERR_NULL_ARGUMENT, "shape is null");
    if (int rc = check_dtype(dtype)) return rc;
    if (int rc = validate_grouped(sh->batch, sh->q_heads, sh->kv_heads, sh->seq_len, sh->head_dim))
        return rc;
    if (rot)
        if (int rc = check_rotary(rot->theta, rot->position_offset, sh->head_dim, sh->seq_len))
            return rc;
    if (int rc = check_head_dim(sh->head_dim, dtype)) return rc;
    float scale;
    if (int rc = resolve_scale(cfg, sh->head_dim, &scale)) return rc;
    const uint64_t eb = elem_bytes(dtype);
    const uint64_t qn = sh->batch * sh->q_heads * sh->seq_len * sh->head_dim;
    const uint64_t kvn = sh->batch * sh->kv_heads * sh->seq_len * sh->head_dim;
    fa_packed_layout lay;
    if (int rc = fa_packed_layout_for(qn, sh->batch * sh->q_heads * sh->seq_len, dtype, &lay)) return rc;
    if (check_buffers) {
        if (int rc = check_buffer("Q", q, q_bytes, qn * eb)) return rc;
        if (int rc = check_buffer("K", k, kv_bytes, kvn * eb)) return rc;
        if (int rc = check_buffer("V", v, kv_bytes, kvn * eb)) return rc;
        if (int rc = check_buffer("O|LSE", out_lse, out_bytes, lay.combined_bytes)) return rc;
    }
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    if (layout) *layout = lay;

    j = PrefillJob{};
    j.dt = (Dtype)dtype;
    j.dtype = dtype;
    fa::PrefillArgs& a = j.a;
    const int64_t S = (int64_t)sh->seq_len, D = (int64_t)sh->head_dim;
    a.q = q; a.k = k; a.v = v;
    a.o = out_lse;
    a.lse = (float*)((uint8_t*)out_lse + lay.lse_byte_offset);
    a.q_sb = (int64_t)sh->q_heads * S * D; a.q_sh = S * D; a.q_ss = D;
    a.k_sb = (int64_t)sh->kv_heads * S * D; a.k_sh = S * D; a.k_ss = D;
    a.o_sb = a.q_sb; a.o_sh = a.q_sh; a.o_ss = a.q_ss;
    a.lse_sb = (int64_t)sh->q_heads * S; a.lse_sh = S;
    a.batch = (int)sh->batch; a.q_heads = (int)sh->q_heads; a.kv_heads = (int)sh->kv_heads;
    a.group = (int)(sh->q_heads / sh->kv_heads);
    a.q_len = (int)S; a.kv_len = (int)S; a.head_dim = (int)D;
    a.causal = cfg && cfg->causal; a.causal_offset = 0;
    a.scale = scale;
    if (rot) {
        j.rope = true;
        j.theta = rot->theta;
        a.rope_q = 1; a.rope_k = 1;
        a.q_rope_offset = (int)rot->position_offset;
        a.kv_rope_offset = (int)rot->position_offset;
        j.max_pos = rot->position_offset + sh->seq_len;
        j.kv_bytes = kvn * eb;
        j.k_rows = sh->batch * sh->kv_heads * sh->seq_len;
        j.k_heads = 1;
        j.k_period = sh->seq_len;
    }
    return FA_OK;
}

}  // namespace

// A contiguous grouped forward with its buffers, shape, configuration and variant resolved and
// its device memory (RoPE table, K rotation workspace) owned, so a launch only enqueues.
struct fa_prepared_forward {
    fa_ctx* ctx = nullptr;
    PrefillRun run;
    fa_packed_layout layout{};
};

extern "C" {

int fa_forward_gqa_rope(fa_ctx* ctx, const void* q, size_t q_bytes, const void* k,
                        const void* v, size_t kv_bytes, void* out_lse, size_t out_bytes,
                        const fa_grouped_shape* sh, const fa_config* cfg, const fa_rotary* rot,
                        int dtype) {
    PrefillJob j;
    if (int rc = build_gqa_job(ctx, q, q_bytes, k, v, kv_bytes, out_lse, out_bytes, sh, cfg, rot,
                               dtype, j, nullptr))
        return rc;
    begin_call(ctx);
    if (int rc = set_device(ctx)) return rc;
    if (int rc = run_prefill(ctx, j)) return rc;
    return ok();
}

// Passive telemetry (WgpuFlatAttention::runtime_telemetry src/wgpu_backend.rs): the record a
// one-shot forward of this shape would leave, built on the host with no device work.
int fa_forward_gqa_rope_telemetry(fa_ctx* ctx, const fa_grouped_shape* sh, const fa_config* cfg,
                                  const fa_rotary* rot, int dtype, fa_telemetry* out) {
    if (!out) return fail(FA_ERR_NULL_ARGUMENT, "output is null");
    PrefillJob j;
    if (int rc = build_gqa_job(ctx, nullptr, 0, nullptr, nullptr, 0, nullptr, 0, sh, cfg, rot,
                               dtype, j, nullptr, false))
        return rc;
    const PrefillChoice c = choose_prefill(ctx, j);
    uint32_t allocs;
    uint64_t bytes;
    predict_prefill_allocs(ctx, j, c, &allocs, &bytes);
    fa::PrefillArgs a = j.a;  // the arguments the prefill kernel would receive
    if (c.prerot) a.rope_k = 0;
    if (c.split_qk) a.split_qk = 1;
    if (c.prec64) a.k_lo = (const void*)(uintptr_t)16;  // stands for the residual the call writes
    a.a64 = ctx->prefill_kernel_policy != 0;
    a.rope_rows = (int)j.max_pos;
    if (j.rope) a.rope_table = (const float2*)(uintptr_t)16;  // stands for the table the call builds
    describe_prefill(ctx, j, a, c.prerot, 1u + c.prerot, allocs, bytes, out);
    return ok();
}

int fa_forward_mha_telemetry(fa_ctx* ctx, const fa_attention_shape* shape, const fa_config* cfg,
                             int dtype, fa_telemetry* out) {
    if (!shape) return fail(FA_ERR_NULL_ARGUMENT, "shape is null");
    fa_grouped_shape g{shape->batch, shape->heads, shape->heads, shape->seq_len, shape->head_dim};
    return fa_forward_gqa_rope_telemetry(ctx, &g, cfg, nullptr, dtype, out);
}

int fa_prepare_gqa_rope(fa_ctx* ctx, const void* q, size_t q_bytes, const void* k,
                        const void* v, size_t kv_bytes, void* out_lse, size_t out_bytes,
                        const fa_grouped_shape* sh, const fa_config* cfg, const fa_rotary* rot,
                        int dtype, fa_prepared_forward** out) {
    if (!out) return fail(FA_ERR_NULL_ARGUMENT, "output handle is null");
    *out = nullptr;
    PrefillJob j;
    fa_packed_layout lay;
    if (int rc = build_gqa_job(ctx, q, q_bytes, k, v, kv_bytes, out_lse, out_bytes, sh, cfg, rot,
                               dtype, j, &lay))
        return rc;
    if (int rc = set_device(ctx)) return rc;
    auto* p = new fa_prepared_forward();
    p->ctx = ctx;
    p->layout = lay;
    if (int rc = resolve_prefill(ctx, j, true, &p->run)) {
        (void)hipStreamSynchronize(ctx->stream);  // error path: the table build may be in flight
        fa_prepared_forward_destroy(p);
        return rc;
    }
    *out = p;
    return ok();
}

int fa_prepare_mha(fa_ctx* ctx, const void* q, const void* k, const void* v, size_t in_bytes,
                   void* out_lse, size_t out_bytes, const fa_attention_shape* shape,
                   const fa_config* config, int dtype, fa_prepared_forward** out) {
    if (!shape) return fail(FA_ERR_NULL_ARGUMENT, "shape is null");
    fa_grouped_shape g{shape->batch, shape->heads, shape->heads, shape->seq_len, shape->head_dim};
    return fa_prepare_gqa_rope(ctx, q, in_bytes, k, v, in_bytes, out_lse, out_bytes, &g, config,
                               nullptr, dtype, out);
}

int fa_launch_prepared(fa_ctx* ctx, const fa_prepared_forward* p) {
    if (!ctx || !p) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (p->ctx != ctx)
        return fail(FA_ERR_FOREIGN_BUFFER, "prepared forward belongs to another context");
    begin_call(ctx);
    if (int rc = set_device(ctx)) return rc;
    if (int rc = enqueue_prefill(ctx, p->run)) return rc;
    return ok();
}

int fa_prepared_forward_layout(const fa_prepared_forward* p, fa_packed_layout* out) {
    if (!p || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    *out = p->layout;
    return ok();
}

int fa_prepared_forward_destroy(fa_prepared_forward* p) {
    if (!p) return ok();
    if (p->ctx && p->ctx->capturing)
        return refuse_in_capture(p->ctx, "release (it waits for the stream)");
    (void)hipSetDevice(p->ctx->device);
    (void)hipStreamSynchronize(p->ctx->stream);
    if (p->run.table) (void)hipFree(p->run.table);
    if (p->run.ws) (void)hipFree(p->run.ws);
    delete p;
    return ok();
}

int fa_forward_mha(fa_ctx* ctx, const void* q, const void* k, const void* v, size_t in_bytes,
                   void* out_lse, size_t out_bytes, const fa_attention_shape* shape,
                   const fa_config* config, int dtype) {
    if (!shape) return fail(FA_ERR_NULL_ARGUMENT, "shape is null");
    fa_grouped_shape g{shape->batch, shape->heads, shape->heads, shape->seq_len, shape->head_dim};
    return fa_forward_gqa_rope(ctx, q, in_bytes, k, v, in_bytes, out_lse, out_bytes, &g, config,
                               nullptr, dtype);
}

}  // extern "C"

namespace {

// AsymmetricGroupedAttentionShape::validate (zero dimensions, head grouping, overflow).
int check_asymmetric_shape(const fa_asymmetric_shape* sh) {
    if (!sh->batch || !sh->q_heads || !sh->kv_heads || !sh->query_len || !sh->kv_len ||
        !sh->head_dim)
        return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
    if (sh->q_heads % sh->kv_heads)
        return fail(FA_ERR_INVALID_HEAD_GROUPING,
                    "q_heads (%llu) must be exactly divisible by kv_heads (%llu)",
                    (unsigned long long)sh->q_heads, (unsigned long long)sh->kv_heads);
    return validate_grouped(sh->batch, sh->q_heads, sh->kv_heads,
                            std::max(sh->query_len, sh->kv_len), sh->head_dim);
}

// The remaining checks of encode_with_options src/wgpu_external_asymmetric.rs:291 that precede
// device work: positions, RoPE, head_dim, scale and buffer sizes. Fills the scale and layout.
int check_asymmetric_pass(const fa_asymmetric_shape* sh, const fa_config* cfg,
                          const fa_asymmetric_rotary* rot, int dtype, const void* q,
                          size_t q_bytes, const void* k, const void* v, size_t kv_bytes,
                          const void* out_lse, size_t out_bytes, float* scale,
                          fa_packed_layout* lay) {
    // (written so that a position near the top of the u64 range cannot wrap past the test)
    if (sh->query_len > kI32 || sh->query_position_offset > kI32 - sh->query_len)
        return fail(FA_ERR_POSITION_OVERFLOW, "rotary position offset overflows the index space");
    if (rot) {
        if (int rc = check_rotary(rot->theta, rot->query_position_offset, sh->head_dim, sh->query_len))
            return rc;
        if (int rc = check_rotary(rot->theta, rot->kv_position_offset, sh->head_dim, sh->kv_len))
            return rc;
    }
    if (int rc = check_head_dim(sh->head_dim, dtype)) return rc;
    if (int rc = resolve_scale(cfg, sh->head_dim, scale)) return rc;
    const uint64_t eb = elem_bytes(dtype);
    const uint64_t qn = sh->batch * sh->query_len * sh->q_heads * sh->head_dim;
    const uint64_t kvn = sh->batch * sh->kv_len * sh->kv_heads * sh->head_dim;
    if (int rc = fa_packed_layout_for(qn, sh->batch * sh->q_heads * sh->query_len, dtype, lay))
        return rc;
    if (int rc = check_buffer("Q", q, q_bytes, qn * eb)) return rc;
    if (int rc = check_buffer("K", k, kv_bytes, kvn * eb)) return rc;
    if (int rc = check_buffer("V", v, kv_bytes, kvn * eb)) return rc;
    return check_buffer("O|LSE", out_lse, out_bytes, lay->combined_bytes);
}

}  // namespace

extern "C" {

int fa_forward_projection_asymmetric(fa_ctx* ctx, const void* q, size_t q_bytes, const void* k,
                                     const void* v, size_t kv_bytes, void* out_lse,
                                     size_t out_bytes, const fa_asymmetric_shape* sh,
                                     const fa_config* cfg, const fa_asymmetric_rotary* rot,
                                     int32_t rotate_k, int dtype) {
    if (!sh) return fail(FA_ERR_NULL_ARGUMENT, "shape is null");
    if (int rc = check_dtype(dtype)) return rc;
    if (int rc = check_asymmetric_shape(sh)) return rc;
    float scale;
    fa_packed_layout lay;
    if (int rc = check_asymmetric_pass(sh, cfg, rot, dtype, q, q_bytes, k, v, kv_bytes, out_lse,
                                       out_bytes, &scale, &lay))
        return rc;
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    begin_call(ctx);
    if (int rc = set_device(ctx)) return rc;

    const uint64_t eb = elem_bytes(dtype);
    const uint64_t kvn = sh->batch * sh->kv_len * sh->kv_heads * sh->head_dim;
    PrefillJob j{};
    j.dt = (Dtype)dtype;
    j.dtype = dtype;
    fa::PrefillArgs& a = j.a;
    const int64_t D = (int64_t)sh->head_dim, QW = (int64_t)sh->q_heads * D,
                  KW = (int64_t)sh->kv_heads * D;
    a.q = q; a.k = k; a.v = v;
    a.o = out_lse;
    a.lse = (float*)((uint8_t*)out_lse + lay.lse_byte_offset);
    a.q_sb = (int64_t)sh->query_len * QW; a.q_sh = D; a.q_ss = QW;
    a.k_sb = (int64_t)sh->kv_len * KW; a.k_sh = D; a.k_ss = KW;
    a.o_sb = a.q_sb; a.o_sh = a.q_sh; a.o_ss = a.q_ss;
    a.lse_sb = (int64_t)sh->q_heads * sh->query_len; a.lse_sh = (int64_t)sh->query_len;
    a.batch = (int)sh->batch; a.q_heads = (int)sh->q_heads; a.kv_heads = (int)sh->kv_heads;
    a.group = (int)(sh->q_heads / sh->kv_heads);
    a.q_len = (int)sh->query_len; a.kv_len = (int)sh->kv_len; a.head_dim = (int)D;
    a.causal = cfg && cfg->causal;
    a.causal_offset = (int)sh->query_position_offset;
    a.scale = scale;
    if (rot) {
        j.rope = true;
        j.theta = rot->theta;
        a.rope_q = 1;
        a.rope_k = rotate_k ? 1 : 0;
        a.q_rope_offset = (int)rot->query_position_offset;
        a.kv_rope_offset = (int)rot->kv_position_offset;
        j.max_pos = std::max(rot->query_position_offset + sh->query_len,
                             rot->kv_position_offset + sh->kv_len);
        j.kv_bytes = kvn * eb;
        j.k_rows = sh->batch * sh->kv_len;
        j.k_heads = sh->kv_heads;
        j.k_period = sh->kv_len;
    }
    if (int rc = run_prefill(ctx, j)) return rc;
    return ok();
}

// ExternalVariableProjectionRotaryGroupedPipeline::encode src/wgpu_external_variable.rs:138 with
// the checks of validate_dispatch :229 in their order. Q/K/V/O keep the padded projection layout;
// sequence b attends over its active rows only (padded K/V rows are never read) and its padded
// query rows get O = 0, LSE = -inf. Q is rotated at meta[b].query_rope_position_offset + t, K at
// kv_position_offset + key; causal masking uses meta[b].query_position_offset + t.
int fa_forward_projection_variable(fa_ctx* ctx, const void* q, size_t q_bytes, const void* k,
                                   const void* v, size_t kv_bytes, void* out_lse,
                                   size_t out_bytes, const fa_asymmetric_shape* sh,
                                   const fa_variable_sequence* meta, uint64_t n_meta,
                                   const fa_config* cfg, float theta, uint64_t kv_position_offset,
                                   int dtype) {
    if (!sh) return fail(FA_ERR_NULL_ARGUMENT, "shape is null");
    if (int rc = check_dtype(dtype)) return rc;
    if (!sh->batch || !sh->q_heads || !sh->kv_heads || !sh->query_len || !sh->kv_len ||
        !sh->head_dim)
        return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
    if (sh->q_heads % sh->kv_heads)
        return fail(FA_ERR_INVALID_HEAD_GROUPING,
                    "q_heads (%llu) must be exactly divisible by kv_heads (%llu)",
                    (unsigned long long)sh->q_heads, (unsigned long long)sh->kv_heads);
    if (int rc = validate_grouped(sh->batch, sh->q_heads, sh->kv_heads,
                                  std::max(sh->query_len, sh->kv_len), sh->head_dim))
        return rc;
    if (n_meta != sh->batch)
        return fail(FA_ERR_LENGTH_MISMATCH,
                    "active sequence metadata contains %llu elements, expected %llu",
                    (unsigned long long)n_meta, (unsigned long long)sh->batch);
    if (n_meta && !meta) return fail(FA_ERR_NULL_ARGUMENT, "metadata is null");
    uint64_t max_pos = 0;
    std::vector<int32_t> m(4 * sh->batch);
    for (uint64_t b = 0; b < sh->batch; ++b) {
        const fa_variable_sequence& e = meta[b];
        if (!e.active_query_len || !e.active_kv_len)
            return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
        if (e.active_query_len > sh->query_len)
            return fail(FA_ERR_LENGTH_MISMATCH, "active query length contains %llu elements, expected %llu",
                        (unsigned long long)e.active_query_len, (unsigned long long)sh->query_len);
        if (e.active_kv_len > sh->kv_len)
            return fail(FA_ERR_LENGTH_MISMATCH, "active KV length contains %llu elements, expected %llu",
                        (unsigned long long)e.active_kv_len, (unsigned long long)sh->kv_len);
        // positions must fit the kernels' i32 index space (the reference bounds them by u32)
        const uint64_t causal_end = e.query_position_offset + e.active_query_len;
        const uint64_t q_rope_end = e.query_rope_position_offset + e.active_query_len;
        const uint64_t kv_rope_end = kv_position_offset + e.active_kv_len;
        if (causal_end < e.query_position_offset || causal_end > kI32 ||
            q_rope_end < e.query_rope_position_offset || q_rope_end > kI32 ||
            kv_rope_end < kv_position_offset || kv_rope_end > kI32)
            return fail(FA_ERR_POSITION_OVERFLOW, "rotary position offset overflows the index space");
        if (int rc = check_rotary(theta, e.query_rope_position_offset, sh->head_dim, e.active_query_len))
            return rc;
        if (int rc = check_rotary(theta, kv_position_offset, sh->head_dim, e.active_kv_len))
            return rc;
        m[4 * b + 0] = (int32_t)e.active_query_len;
        m[4 * b + 1] = (int32_t)e.active_kv_len;
        m[4 * b + 2] = (int32_t)e.query_position_offset;
        m[4 * b + 3] = (int32_t)e.query_rope_position_offset;
        max_pos = std::max(max_pos, std::max(q_rope_end, kv_rope_end));
    }
    if (int rc = check_head_dim(sh->head_dim, dtype)) return rc;
    const uint64_t eb = elem_bytes(dtype);
    const uint64_t qn = sh->batch * sh->query_len * sh->q_heads * sh->head_dim;
    const uint64_t kvn = sh->batch * sh->kv_len * sh->kv_heads * sh->head_dim;
    fa_packed_layout lay;
    if (int rc = fa_packed_layout_for(qn, sh->batch * sh->q_heads * sh->query_len, dtype, &lay))
        return rc;
    if (int rc = check_buffer("Q", q, q_bytes, qn * eb)) return rc;
    if (int rc = check_buffer("K", k, kv_bytes, kvn * eb)) return rc;
    if (int rc = check_buffer("V", v, kv_bytes, kvn * eb)) return rc;
    if (int rc = check_buffer("O|LSE", out_lse, out_bytes, lay.combined_bytes)) return rc;
    float scale;
    if (int rc = resolve_scale(cfg, sh->head_dim, &scale)) return rc;
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    begin_call(ctx);
    if (int rc = set_device(ctx)) return rc;

    PrefillJob j{};
    j.dt = (Dtype)dtype;
    j.dtype = dtype;
    fa::PrefillArgs& a = j.a;
    const int64_t D = (int64_t)sh->head_dim, QW = (int64_t)sh->q_heads * D,
                  KW = (int64_t)sh->kv_heads * D;
    a.q = q; a.k = k; a.v = v;
    a.o = out_lse;
    a.lse = (float*)((uint8_t*)out_lse + lay.lse_byte_offset);
    a.q_sb = (int64_t)sh->query_len * QW; a.q_sh = D; a.q_ss = QW;
    a.k_sb = (int64_t)sh->kv_len * KW; a.k_sh = D; a.k_ss = KW;
    a.o_sb = a.q_sb; a.o_sh = a.q_sh; a.o_ss = a.q_ss;
    a.lse_sb = (int64_t)sh->q_heads * sh->query_len; a.lse_sh = (int64_t)sh->query_len;
    a.batch = (int)sh->batch; a.q_heads = (int)sh->q_heads; a.kv_heads = (int)sh->kv_heads;
    a.group = (int)(sh->q_heads / sh->kv_heads);
    a.q_len = (int)sh->query_len; a.kv_len = (int)sh->kv_len; a.head_dim = (int)D;
    a.causal = cfg && cfg->causal;
    a.scale = scale;
    j.rope = true;
    j.theta = theta;
    a.rope_q = 1;
    a.rope_k = 1;
    a.kv_rope_offset = (int)kv_position_offset;
    j.max_pos = max_pos;
    j.kv_bytes = kvn * eb;
    j.k_rows = sh->batch * sh->kv_len;
    j.k_heads = sh->kv_heads;
    j.k_period = sh->kv_len;
    if (int rc = upload_meta(ctx, m.data(), m.size(), &a.var_meta)) return rc;
    if (int rc = run_prefill(ctx, j)) return rc;
    return ok();
}

int fa_chunked_prefill(fa_ctx* ctx, const void* q, size_t q_bytes, const void* k, const void* v,
                       size_t kv_bytes, void* out_lse, size_t out_bytes,
                       const fa_grouped_shape* sh, const fa_config* cfg, const fa_rotary* rot,
                       uint64_t query_chunk_size, int dtype) {
    if (!sh || !rot) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (query_chunk_size == 0)
        return fail(FA_ERR_ZERO_QUERY_CHUNK_SIZE,
                    "chunked projection prefill requires a non-zero query chunk size");
    if (int rc = validate_grouped(sh->batch, sh->q_heads, sh->kv_heads, sh->seq_len, sh->head_dim))
        return rc;
    if (int rc = check_rotary(rot->theta, rot->position_offset, sh->head_dim, sh->seq_len)) return rc;
    // Every query row's K/V visitation order and online-softmax arithmetic are independent of
    // the chunk it belongs to (src/chunked_projection_prefill.rs:1-7), so all chunks run in one
    // launch whose result is identical for every chunk size.
    fa_asymmetric_shape as{sh->batch, sh->q_heads, sh->kv_heads, sh->seq_len, sh->seq_len,
                           sh->head_dim, 0};
    fa_asymmetric_rotary ar{rot->theta, rot->position_offset, rot->position_offset};
    return fa_forward_projection_asymmetric(ctx, q, q_bytes, k, v, kv_bytes, out_lse, out_bytes,
                                            &as, cfg, &ar, 1, dtype);
}

int fa_kernel_variant_for_shape(fa_ctx* ctx, uint64_t head_dim, int32_t has_rope, int dtype,
                                int32_t* kernel_id) {
    if (!ctx || !kernel_id) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = check_dtype(dtype)) return rc;
    if (int rc = check_head_dim(head_dim, dtype)) return rc;
    *kernel_id = prefill_kernel_id(dtype, has_rope && want_prerotate(ctx, head_dim));
    return ok();
}

}  // extern "C"

// ---------------------------------------------------------------------------- host forwards
namespace {

bool finite16(uint16_t h, int dtype) {
    return dtype == FA_DTYPE_BF16 ? (h & 0x7f80u) != 0x7f80u : (h & 0x7c00u) != 0x7c00u;
}

int validate_host_input(const char* name, const void* data, uint64_t len, uint64_t expected,
                        int dtype) {
    if (!data && len) return fail(FA_ERR_NULL_ARGUMENT, "tensor %s is null", name);
    if (len != expected)
        return fail(FA_ERR_LENGTH_MISMATCH, "tensor %s contains %llu elements, expected %llu", name,
                    (unsigned long long)len, (unsigned long long)expected);
    for (uint64_t i = 0; i < len; ++i) {
        bool fin = dtype == FA_DTYPE_F32 ? std::isfinite(((const float*)data)[i])
                                         : finite16(((const uint16_t*)data)[i], dtype);
        if (!fin)
            return fail(FA_ERR_NON_FINITE_INPUT, "tensor %s contains a non-finite value at index %llu",
                        name, (unsigned long long)i);
    }
    return FA_OK;
}

struct DevBuf {
    void* p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

}  // namespace

extern "C" {

int fa_forward_gqa_rope_host(fa_ctx* ctx, const void* q, const void* k, const void* v,
                             uint64_t q_len, uint64_t k_len, uint64_t v_len,
                             const fa_grouped_shape* sh, const fa_config* cfg,
                             const fa_rotary* rot, int dtype, void* out, float* lse) {
    if (!sh || !out || !lse) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = check_dtype(dtype)) return rc;
    if (int rc = validate_grouped(sh->batch, sh->q_heads, sh->kv_heads, sh->seq_len, sh->head_dim))
        return rc;
    if (rot)
        if (int rc = check_rotary(rot->theta, rot->position_offset, sh->head_dim, sh->seq_len))
            return rc;
    const uint64_t qn = sh->batch * sh->q_heads * sh->seq_len * sh->head_dim;
    const uint64_t kvn = sh->batch * sh->kv_heads * sh->seq_len * sh->head_dim;
    if (int rc = validate_host_input("Q", q, q_len, qn, dtype)) return rc;
    if (int rc = validate_host_input("K", k, k_len, kvn, dtype)) return rc;
    if (int rc = validate_host_input("V", v, v_len, kvn, dtype)) return rc;
    float scale;
    if (int rc = resolve_scale(cfg, sh->head_dim, &scale)) return rc;
    if (int rc = check_head_dim(sh->head_dim, dtype)) return rc;
    const uint64_t eb = elem_bytes(dtype);
    fa_packed_layout lay;
    if (int rc = fa_packed_layout_for(qn, sh->batch * sh->q_heads * sh->seq_len, dtype, &lay)) return rc;
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    if (int rc = set_device(ctx)) return rc;
    DevBuf dq, dk, dv, dout;
    HIP_TRY(hipMalloc(&dq.p, qn * eb));
    HIP_TRY(hipMalloc(&dk.p, kvn * eb));
    HIP_TRY(hipMalloc(&dv.p, kvn * eb));
    HIP_TRY(hipMalloc(&dout.p, lay.combined_bytes));
    HIP_TRY(hipMemcpyAsync(dq.p, q, qn * eb, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipMemcpyAsync(dk.p, k, kvn * eb, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipMemcpyAsync(dv.p, v, kvn * eb, hipMemcpyHostToDevice, ctx->stream));
    int rc = fa_forward_gqa_rope(ctx, dq.p, qn * eb, dk.p, dv.p, kvn * eb, dout.p,
                                 lay.combined_bytes, sh, cfg, rot, dtype);
    if (rc) {
        (void)hipStreamSynchronize(ctx->stream);
        return rc;
    }
    ctx->last.temporary_allocation_count += 4;
    ctx->last.temporary_allocation_bytes += 2 * qn * eb + 2 * kvn * eb;
    HIP_TRY(hipMemcpyAsync(out, dout.p, lay.output_bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipMemcpyAsync(lse, (uint8_t*)dout.p + lay.lse_byte_offset, lay.lse_elements * 4,
                           hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return ok();
}

int fa_forward_mha_host(fa_ctx* ctx, const void* q, const void* k, const void* v,
                        uint64_t q_len, uint64_t k_len, uint64_t v_len,
                        const fa_attention_shape* shape, const fa_config* config, int dtype,
                        void* out, float* lse) {
    if (!shape) return fail(FA_ERR_NULL_ARGUMENT, "shape is null");
    if (!shape->batch || !shape->heads || !shape->seq_len || !shape->head_dim)
        return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
    fa_grouped_shape g{shape->batch, shape->heads, shape->heads, shape->seq_len, shape->head_dim};
    return fa_forward_gqa_rope_host(ctx, q, k, v, q_len, k_len, v_len, &g, config, nullptr, dtype,
                                    out, lse);
}

}  // extern "C"

// ---------------------------------------------------------------------------- paged KV table
struct fa_kv_table {
    uint64_t page_size = 0, physical_pages = 0, live = 0, generation = 0;
    std::vector<std::pair<uint64_t, uint64_t>> logical;  // (physical page, generation)
    std::vector<uint64_t> free_pages;                     // stack, lowest id on top
};

namespace {

int table_capacity(const fa_kv_table* t, uint64_t* cap) {
    if (!t->page_size || !t->physical_pages)
        return fail(FA_ERR_PAGED_ZERO_DIMENSION, "paged KV dimensions must be non-zero");
    if (mul_ov(t->page_size, t->physical_pages, cap))
        return fail(FA_ERR_CAPACITY_OVERFLOW, "paged KV capacity overflows usize");
    return FA_OK;
}

void fill_free(fa_kv_table* t) {
    t->free_pages.clear();
    t->free_pages.reserve(t->physical_pages);
    for (uint64_t p = t->physical_pages; p-- > 0;) t->free_pages.push_back(p);
}

}  // namespace

extern "C" {

int fa_kv_table_create(uint64_t page_size, uint64_t physical_pages, fa_kv_table** out) {
    if (!out) return fail(FA_ERR_NULL_ARGUMENT, "output pointer is null");
    fa_kv_table tmp;
    tmp.page_size = page_size;
    tmp.physical_pages = physical_pages;
    uint64_t cap;
    if (int rc = table_capacity(&tmp, &cap)) return rc;
    fa_kv_table* t = new fa_kv_table(tmp);
    fill_free(t);
    *out = t;
    return ok();
}

int fa_kv_table_destroy(fa_kv_table* t) {
    delete t;
    return ok();
}

int fa_kv_table_clone(const fa_kv_table* t, fa_kv_table** out) {
    if (!t || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    *out = new fa_kv_table(*t);
    return ok();
}

int fa_kv_table_append(fa_kv_table* t, uint64_t tokens) {
    if (!t) return fail(FA_ERR_NULL_ARGUMENT, "table is null");
    if (tokens == 0) return ok();
    if (t->live > std::numeric_limits<uint64_t>::max() - tokens)
        return fail(FA_ERR_CAPACITY_OVERFLOW, "paged KV capacity overflows usize");
    const uint64_t new_len = t->live + tokens;
    uint64_t cap;
    if (int rc = table_capacity(t, &cap)) return rc;
    if (new_len > cap)
        return fail(FA_ERR_CAPACITY_EXCEEDED, "paged KV append requires %llu tokens, capacity is %llu",
                    (unsigned long long)new_len, (unsigned long long)cap);
    const uint64_t required = (new_len + t->page_size - 1) / t->page_size;
    while (t->logical.size() < required) {
        const uint64_t p = t->free_pages.back();
        t->free_pages.pop_back();
        t->logical.push_back({p, t->generation});
    }
    t->live = new_len;
    return ok();
}

int fa_kv_table_address(const fa_kv_table* t, uint64_t logical_token, fa_kv_address* out) {
    if (!t || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (logical_token >= t->live) return fail(FA_ERR_EMPTY_TABLE, "logical token is not mapped");
    const uint64_t lp = logical_token / t->page_size;
    if (lp >= t->logical.size() || t->logical[lp].second != t->generation)
        return fail(FA_ERR_EMPTY_TABLE, "logical token is not mapped");
    out->physical_page = t->logical[lp].first;
    out->offset_in_page = logical_token % t->page_size;
    out->generation = t->logical[lp].second;
    return ok();
}

int fa_kv_table_telemetry(const fa_kv_table* t, fa_kv_telemetry* out) {
    if (!t || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    uint64_t cap;
    if (int rc = table_capacity(t, &cap)) return rc;
    uint64_t alloc;
    if (mul_ov((uint64_t)t->logical.size(), t->page_size, &alloc))
        return fail(FA_ERR_CAPACITY_OVERFLOW, "paged KV capacity overflows usize");
    out->live_tokens = t->live;
    out->capacity_tokens = cap;
    out->mapped_pages = t->logical.size();
    out->free_pages = t->free_pages.size();
    out->internal_fragmentation_tokens = alloc - t->live;
    out->generation = t->generation;
    return ok();
}

int fa_kv_table_reset(fa_kv_table* t) {
    if (!t) return fail(FA_ERR_NULL_ARGUMENT, "table is null");
    if (t->generation == std::numeric_limits<uint64_t>::max())
        return fail(FA_ERR_GENERATION_OVERFLOW, "paged KV generation counter overflowed");
    t->generation += 1;
    t->live = 0;
    t->logical.clear();
    fill_free(t);
    return ok();
}

uint64_t fa_kv_table_len(const fa_kv_table* t) { return t ? t->live : 0; }

int fa_kv_table_block_row(const fa_kv_table* t, int32_t* out, uint64_t capacity, uint64_t* count) {
    if (!t || !count) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (t->live == 0 || t->logical.empty())
        return fail(FA_ERR_EMPTY_TABLE, "paged decode requires at least one live KV token");
    *count = t->logical.size();
    if (!out) return ok();
    if (capacity < t->logical.size())
        return fail(FA_ERR_BUFFER_TOO_SMALL, "block row holds %llu entries, requires %llu",
                    (unsigned long long)capacity, (unsigned long long)t->logical.size());
    for (size_t i = 0; i < t->logical.size(); ++i) {
        if (t->logical[i].first > kI32)
            return fail(FA_ERR_INDEX_SPACE_EXCEEDED, "physical page %llu exceeds the i32 index space",
                        (unsigned long long)t->logical[i].first);
        out[i] = (int32_t)t->logical[i].first;
    }
    return ok();
}

}  // extern "C"

// ---------------------------------------------------------------------------- paged cache
struct fa_paged_cache {
    fa_ctx* ctx = nullptr;
    fa_kv_table table;
    uint64_t kv_heads = 0, head_dim = 0, row_bytes = 0, tensor_bytes = 0;
    int dtype = 0;
    void* k = nullptr;
    void* v = nullptr;
};

extern "C" {

int fa_paged_cache_create(fa_ctx* ctx, uint64_t page_size, uint64_t physical_pages,
                          uint64_t kv_heads, uint64_t head_dim, int dtype, fa_paged_cache** out) {
    if (!ctx || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = check_dtype(dtype)) return rc;
    if (!kv_heads || !head_dim)
        return fail(FA_ERR_ZERO_DIMENSION, "paged resident KV dimensions must be non-zero");
    fa_kv_table* t = nullptr;
    if (int rc = fa_kv_table_create(page_size, physical_pages, &t)) return rc;
    uint64_t row_el, row_b, cap, bytes;
    if (mul_ov(kv_heads, head_dim, &row_el) || mul_ov(row_el, elem_bytes(dtype), &row_b) ||
        mul_ov(page_size, physical_pages, &cap) || mul_ov(cap, row_b, &bytes)) {
        delete t;
        return fail(FA_ERR_SHAPE_OVERFLOW, "paged resident KV shape overflows the address space");
    }
    if (int rc = set_device(ctx)) {
        delete t;
        return rc;
    }
    fa_paged_cache* c = new fa_paged_cache();
    c->ctx = ctx;
    c->table = *t;
    delete t;
    c->kv_heads = kv_heads;
    c->head_dim = head_dim;
    c->row_bytes = row_b;
    c->tensor_bytes = bytes;
    c->dtype = dtype;
    if (hipMalloc(&c->k, bytes) != hipSuccess || hipMalloc(&c->v, bytes) != hipSuccess) {
        if (c->k) (void)hipFree(c->k);
        delete c;
        return fail(FA_ERR_HIP, "paged resident KV requires %llu bytes per tensor",
                    (unsigned long long)bytes);
    }
    *out = c;
    return ok();
}

int fa_paged_cache_destroy(fa_paged_cache* c) {
    if (!c) return ok();
    if (c->ctx && c->ctx->capturing)
        return refuse_in_capture(c->ctx, "release (it waits for the stream)");
    (void)hipSetDevice(c->ctx->device);
    (void)hipStreamSynchronize(c->ctx->stream);
    (void)hipFree(c->k);
    (void)hipFree(c->v);
    delete c;
    return ok();
}

int fa_paged_cache_append(fa_paged_cache* c, const void* k_src, const void* v_src,
                          size_t src_bytes, uint64_t append_len, const fa_rotary* rot,
                          uint64_t* new_len) {
    if (!c) return fail(FA_ERR_NULL_ARGUMENT, "cache is null");
    fa_ctx* ctx = c->ctx;
    begin_call(ctx);
    if (append_len == 0)
        return fail(FA_ERR_ZERO_DIMENSION, "paged resident KV dimensions must be non-zero");
    uint64_t need;
    if (mul_ov(append_len, c->row_bytes, &need))
        return fail(FA_ERR_SHAPE_OVERFLOW, "paged resident KV shape overflows the address space");
    if (int rc = check_buffer("K", k_src, src_bytes, need)) return rc;
    if (int rc = check_buffer("V", v_src, src_bytes, need)) return rc;
    const float2* table = nullptr;
    if (rot) {
        if (int rc = check_rotary(rot->theta, rot->position_offset, c->head_dim,
                                  c->table.live + append_len))
            return rc;
        if (c->head_dim % 8 != 0)
            return fail(FA_ERR_UNSUPPORTED_HEAD_DIM,
                        "rotate-on-append needs head_dim %% 8 == 0, got %llu",
                        (unsigned long long)c->head_dim);
    }
    fa_kv_table staged = c->table;
    const uint64_t old_len = staged.live;
    if (int rc = fa_kv_table_append(&staged, append_len)) return rc;
    if (int rc = set_device(ctx)) return rc;
    if (rot) {
        if (int rc = ensure_rope(ctx, rot->theta, c->head_dim,
                                 rot->position_offset + staged.live, &table))
            return rc;
    }
    uint32_t dispatches = 0;
    uint64_t logical = old_len, src_row = 0;
    while (logical < staged.live) {
        fa_kv_address addr;
        if (int rc = fa_kv_table_address(&staged, logical, &addr)) return rc;
        const uint64_t rows = std::min(staged.page_size - addr.offset_in_page, staged.live - logical);
        const uint64_t prow = addr.physical_page * staged.page_size + addr.offset_in_page;
        const uint64_t so = src_row * c->row_bytes, dof = prow * c->row_bytes;
        if (dof + rows * c->row_bytes > c->tensor_bytes)
            return fail(FA_ERR_SHAPE_OVERFLOW, "paged resident KV shape overflows the address space");
        if (rot) {
            begin_span(ctx);
            fa::launch_rotate_rows((Dtype)c->dtype, (const uint8_t*)k_src + so, (uint8_t*)c->k + dof,
                                   (int)rows, (int)c->kv_heads, (int)c->head_dim, (int64_t)kI32,
                                   table, (int)(rot->position_offset + logical), ctx->stream);
            end_span(ctx, FA_KERNEL_ROPE_ROTATE);
            HIP_TRY(hipGetLastError());
        } else {
            HIP_TRY(hipMemcpyAsync((uint8_t*)c->k + dof, (const uint8_t*)k_src + so,
                                   rows * c->row_bytes, hipMemcpyDeviceToDevice, ctx->stream));
        }
        HIP_TRY(hipMemcpyAsync((uint8_t*)c->v + dof, (const uint8_t*)v_src + so, rows * c->row_bytes,
                               hipMemcpyDeviceToDevice, ctx->stream));
        dispatches += 2;
        logical += rows;
        src_row += rows;
    }
    c->table = staged;
    if (new_len) *new_len = staged.live;
    unsigned grid[3] = {(unsigned)append_len, 1, 1};
    record(ctx, FA_KERNEL_PAGED_APPEND, "paged append (per-page copies)", 0,
           (uint32_t)c->table.page_size, grid, 0, dispatches, 1, nullptr);
    return ok();
}

int fa_paged_cache_reset(fa_paged_cache* c) {
    if (!c) return fail(FA_ERR_NULL_ARGUMENT, "cache is null");
    return fa_kv_table_reset(&c->table);
}

const fa_kv_table* fa_paged_cache_table(const fa_paged_cache* c) { return c ? &c->table : nullptr; }
void* fa_paged_cache_k(fa_paged_cache* c) { return c ? c->k : nullptr; }
void* fa_paged_cache_v(fa_paged_cache* c) { return c ? c->v : nullptr; }
size_t fa_paged_cache_bytes(const fa_paged_cache* c) { return c ? (size_t)c->tensor_bytes : 0; }

}  // extern "C"

// ---------------------------------------------------------------------------- paged decode
struct fa_decode_plan {
    fa_ctx* ctx = nullptr;
    uint64_t n_seqs = 0, max_pages = 0, page_size = 0, physical_pages = 0;
    uint64_t q_heads = 0, kv_heads = 0, head_dim = 0;
    int dtype = 0;
    float scale = 0.0f, theta = 0.0f;
    std::vector<int32_t> ctx_lens;
    uint64_t split_req = 0;     // requested segment length (0 = equal ranges per wave)
    uint64_t split_tokens = 0;  // longest segment of the current work list
    uint64_t n_work = 0;        // segments
    uint64_t n_waves = 0, n_slots = 0, units = 0;
    int grouped = 0;  // > 0: head-grouped workgroups of this many waves (one per unit)
    uint64_t max_pos = 0;
    // device
    int32_t* d_bt = nullptr;
    int32_t* d_ctx = nullptr;
    int32_t* d_qpos = nullptr;
    int32_t* d_work = nullptr;  // [seg (5 per segment) | wave_off | unit_part]
    float* d_part = nullptr;    // partial O then (m, l)
    uint64_t part_bytes = 0;
    uint64_t work_cap = 0;
};

namespace {

// A split may touch at most 64 pages (one block-table entry per lane of the decode wave).
uint64_t max_split_tokens(uint64_t page_size) {
    const uint64_t t = (63 * page_size + 1) / 16 * 16;
    return std::max<uint64_t>(16, t);
}

// Work list of a decode plan. A unit is (kv head, chunk of <= 16 query heads); the key space
// of every (sequence, unit) is laid end to end, each unit padded to a multiple of 16 keys, and
// cut into segments:
//  * automatic (split_req == 0): one equal range of whole 16-key steps per resident wave, so
//    every wave streams the same number of K/V bytes (segments also end at unit boundaries and
//    after max_split_tokens keys);
//  * split_req = x: every unit cut every x keys, segments dealt to the resident waves in turn.
// Units covered by one segment are finalised by the split kernel; the others get one partial
// slot per segment, merged by the combine kernel.
int compute_work(fa_decode_plan* p, std::vector<int32_t>* all_out) {
    fa_ctx* ctx = p->ctx;
    const uint64_t chunks = (p->q_heads / p->kv_heads + 15) / 16;
    const uint64_t units = p->kv_heads * chunks;
    const uint64_t maxseg = max_split_tokens(p->page_size);
    // Head-grouped mode (16-bit KV, page_size % 16 == 0, automatic split, <= 8 units): one
    // workgroup of `units` waves per segment list, every wave on the same key ranges.
    const bool want_grouped = ctx->decode_grouped_policy != 0;
    p->grouped = (want_grouped && p->split_req == 0 && p->dtype != (int)Dtype::F32 &&
                  p->page_size % 16 == 0 && units <= 8)
                     ? (int)units
                     : 0;
    const int resident = fa::decode_resident_waves(
        (Dtype)p->dtype, (int)p->head_dim, (int)(p->q_heads / p->kv_heads), (int)p->page_size,
        p->grouped);
    const uint64_t G = (uint64_t)std::max(1, resident);
    struct Seg { int32_t s, u, k0, k1, slot; uint64_t wave; };
    std::vector<Seg> segs;
    std::vector<int32_t> unit_part(p->n_seqs * units + 1, 0);
    uint64_t longest = 0;
    if (p->grouped > 0) {
        uint64_t total = 0;
        for (int32_t c : p->ctx_lens) total += ((uint64_t)c + 15) / 16 * 16;
        const uint64_t L = std::max<uint64_t>(16, ((total + G - 1) / G + 15) / 16 * 16);
        uint64_t pos = 0;
        int32_t slot = 0;
        for (uint64_t s = 0; s < p->n_seqs; ++s) {
            const uint64_t c = (uint64_t)p->ctx_lens[s];
            const uint64_t cpad = (c + 15) / 16 * 16;
            const size_t first = segs.size();
            for (uint64_t t = 0; t < cpad;) {
                const uint64_t wave = (pos + t) / L;
                const uint64_t e = std::min(std::min(cpad, (wave + 1) * L - pos), t + maxseg);
                segs.push_back({(int32_t)s, 0, (int32_t)t, (int32_t)std::min(c, e), -1, wave});
                longest = std::max(longest, e - t);
                t = e;
            }
            pos += cpad;
            const int32_t nseg = (int32_t)(segs.size() - first);
            for (uint64_t u = 0; u < units; ++u)
                unit_part[s * units + u] = nseg > 1 ? slot + (int32_t)u * nseg : slot;
            if (nseg > 1) {
                for (int32_t j = 0; j < nseg; ++j) {
                    segs[first + j].u = nseg;
                    segs[first + j].slot = slot + j;
                }
                slot += (int32_t)units * nseg;
            }
        }
        unit_part[p->n_seqs * units] = slot;
        p->n_slots = (uint64_t)slot;
        if (segs.size() > kI32)
            return fail(FA_ERR_DISPATCH_LIMIT, "paged decode requires %llu segments",
                        (unsigned long long)segs.size());
    } else {
    uint64_t total = 0;
    for (int32_t c : p->ctx_lens) total += ((uint64_t)c + 15) / 16 * 16 * units;
    if (p->split_req == 0) {
        const uint64_t L = std::max<uint64_t>(16, ((total + G - 1) / G + 15) / 16 * 16);
        uint64_t pos = 0;
        for (uint64_t s = 0; s < p->n_seqs; ++s) {
            const uint64_t c = (uint64_t)p->ctx_lens[s];
            const uint64_t cpad = (c + 15) / 16 * 16;
            for (uint64_t u = 0; u < units; ++u) {
                for (uint64_t t = 0; t < cpad;) {
                    const uint64_t wave = (pos + t) / L;
                    const uint64_t wave_end = (wave + 1) * L - pos;  // unit-relative
                    const uint64_t e = std::min(std::min(cpad, wave_end), t + maxseg);
                    segs.push_back({(int32_t)s, (int32_t)u, (int32_t)t,
                                    (int32_t)std::min(c, e), -1, wave});
                    longest = std::max(longest, e - t);
                    t = e;
                }
                pos += cpad;
            }
        }
    } else {
        uint64_t i = 0;
        for (uint64_t s = 0; s < p->n_seqs; ++s) {
            const uint64_t c = (uint64_t)p->ctx_lens[s];
            for (uint64_t u = 0; u < units; ++u)
                for (uint64_t t = 0; t < c; t += p->split_req, ++i) {
                    const uint64_t e = std::min(c, t + p->split_req);
                    segs.push_back({(int32_t)s, (int32_t)u, (int32_t)t, (int32_t)e, -1, i % G});
                    longest = std::max(longest, e - t);
                }
        }
    }
    if (segs.size() > kI32)
        return fail(FA_ERR_DISPATCH_LIMIT, "paged decode requires %llu segments",
                    (unsigned long long)segs.size());
    // partial slots: units with more than one segment
    {
        size_t i = 0;
        int32_t slot = 0;
        for (uint64_t su = 0; su < p->n_seqs * units; ++su) {
            unit_part[su] = slot;
            size_t j = i;
            while (j < segs.size() && (uint64_t)segs[j].s * units + segs[j].u == su) ++j;
            if (j - i > 1)
                for (size_t k = i; k < j; ++k) segs[k].slot = slot++;
            i = j;
        }
        unit_part[p->n_seqs * units] = slot;
        p->n_slots = (uint64_t)slot;
    }
    }  // one-wave mode
    // per-wave lists (segments are generated in increasing wave order in the automatic mode)
    uint64_t n_waves = 0;
    for (const Seg& g : segs) n_waves = std::max(n_waves, g.wave + 1);
    std::vector<int32_t> wave_off(n_waves + 1, 0);
    for (const Seg& g : segs) wave_off[g.wave + 1]++;
    for (uint64_t w = 0; w < n_waves; ++w) wave_off[w + 1] += wave_off[w];
    std::vector<int32_t> seg_arr(5 * segs.size());
    {
        std::vector<int32_t> fill(wave_off.begin(), wave_off.end() - 1);
        for (const Seg& g : segs) {
            const int32_t at = fill[g.wave]++;
            seg_arr[5 * at + 0] = g.s;
            seg_arr[5 * at + 1] = g.u;
            seg_arr[5 * at + 2] = g.k0;
            seg_arr[5 * at + 3] = g.k1;
            seg_arr[5 * at + 4] = g.slot;
        }
    }
    p->n_work = segs.size();
    p->n_waves = n_waves;
    p->units = units;
    p->split_tokens = longest;
    const uint64_t need_work = seg_arr.size() + wave_off.size() + unit_part.size();
    std::vector<int32_t>& all = *all_out;
    all.clear();
    all.reserve(need_work);
    all.insert(all.end(), seg_arr.begin(), seg_arr.end());
    all.insert(all.end(), wave_off.begin(), wave_off.end());
    all.insert(all.end(), unit_part.begin(), unit_part.end());
    return FA_OK;
}

// Partial slots hold un-normalised O (16 heads x head_dim) then (m, l) per head.
uint64_t partial_bytes(const fa_decode_plan* p) {
    return std::max<uint64_t>(1, p->n_slots) * 16 * (p->head_dim + 2) * 4;
}

int build_work(fa_decode_plan* p) {
    fa_ctx* ctx = p->ctx;
    std::vector<int32_t> all;
    if (int rc = compute_work(p, &all)) return rc;
    const uint64_t need_work = all.size();
    // (a plan rebuilt by set_split may still be read by launches in flight: a buffer that grows
    // is retired to the context, and the new lists arrive by a stream-ordered copy)
    if (p->work_cap < need_work) {
        void* fresh = nullptr;
        if (int rc = dev_alloc(ctx, &fresh, need_work * 4)) return rc;
        if (p->d_work) ctx->retired.push_back(p->d_work);
        p->d_work = (int32_t*)fresh;
        p->work_cap = need_work;
    }
    if (int rc = stage_upload(ctx, p->d_work, all.data(), need_work * 4)) return rc;
    const uint64_t part = partial_bytes(p);
    if (p->part_bytes < part) {
        void* fresh = nullptr;
        if (int rc = dev_alloc(ctx, &fresh, part)) return rc;
        if (p->d_part) ctx->retired.push_back(p->d_part);
        p->d_part = (float*)fresh;
        p->part_bytes = part;
    }
    return FA_OK;
}

void free_plan(fa_decode_plan* p) {
    if (p->d_bt) (void)hipFree(p->d_bt);
    if (p->d_ctx) (void)hipFree(p->d_ctx);
    if (p->d_qpos) (void)hipFree(p->d_qpos);
    if (p->d_work) (void)hipFree(p->d_work);
    if (p->d_part) (void)hipFree(p->d_part);
    delete p;
}

int check_pages(const int32_t* bt, uint64_t max_pages, uint64_t n_seqs, uint64_t live_len,
                const int32_t* lens, uint64_t page_size, uint64_t physical_pages) {
    for (uint64_t s = 0; s < n_seqs; ++s) {
        const uint64_t len = lens ? (uint64_t)lens[s] : live_len;
        const uint64_t pages = (len + page_size - 1) / page_size;
        if (pages > max_pages)
            return fail(FA_ERR_INDEX_SPACE_EXCEEDED,
                        "sequence %llu needs %llu pages, block table holds %llu",
                        (unsigned long long)s, (unsigned long long)pages,
                        (unsigned long long)max_pages);
        for (uint64_t p = 0; p < pages; ++p) {
            const int32_t id = bt[s * max_pages + p];
            if (id < 0 || (uint64_t)id >= physical_pages)
                return fail(FA_ERR_INVALID_PAGE,
                            "sequence %llu logical page %llu maps to physical page %d outside [0, %llu)",
                            (unsigned long long)s, (unsigned long long)p, id,
                            (unsigned long long)physical_pages);
        }
    }
    return FA_OK;
}

// Arguments of a paged decode (fa_paged_decode_prepare): every check that precedes device work.
// Fills the softmax scale, each query's RoPE position and the table rows they need.
int validate_decode(const int32_t* block_tables, uint64_t max_pages, const int32_t* ctx_lens,
                    const int32_t* q_positions, uint64_t n_seqs, uint64_t page_size,
                    uint64_t physical_pages, uint64_t q_heads, uint64_t kv_heads,
                    uint64_t head_dim, const fa_config* cfg, float theta, int dtype, float* scale,
                    std::vector<int32_t>* qpos_out, uint64_t* max_pos_out) {
    if (!block_tables || !ctx_lens) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = check_dtype(dtype)) return rc;
    if (!n_seqs || !q_heads || !kv_heads || !head_dim || !max_pages)
        return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
    if (!page_size || !physical_pages)
        return fail(FA_ERR_PAGED_ZERO_DIMENSION, "paged KV dimensions must be non-zero");
    if (q_heads % kv_heads)
        return fail(FA_ERR_INVALID_HEAD_GROUPING,
                    "q_heads (%llu) must be exactly divisible by kv_heads (%llu)",
                    (unsigned long long)q_heads, (unsigned long long)kv_heads);
    if (head_dim > kMaxHeadDim)
        return fail(FA_ERR_UNSUPPORTED_HEAD_DIM, "head_dim %llu exceeds portable maximum %llu",
                    (unsigned long long)head_dim, (unsigned long long)kMaxHeadDim);
    if (head_dim % 2)
        return fail(FA_ERR_INVALID_ROTARY_HEAD_DIM,
                    "rotary attention head_dim must be non-zero and even, got %llu",
                    (unsigned long long)head_dim);
    if (head_dim % (dtype == FA_DTYPE_F32 ? 4 : 8))
        return fail(FA_ERR_UNSUPPORTED_HEAD_DIM, "head_dim %llu is not a multiple of %d for %s decode",
                    (unsigned long long)head_dim, dtype == FA_DTYPE_F32 ? 4 : 8, dtype_name(dtype));
    if (!std::isfinite(theta) || theta <= 0.0f)
        return fail(FA_ERR_INVALID_ROTARY_THETA,
                    "paged decode RoPE theta must be finite and positive, got %g", (double)theta);
    if (int rc = resolve_scale(cfg, head_dim, scale)) return rc;
    uint64_t rows, x;
    if (mul_ov(page_size, physical_pages, &rows) || rows > kI32 || max_pages > kI32 ||
        mul_ov(n_seqs, max_pages, &x) || x > (uint64_t)std::numeric_limits<int64_t>::max() / 4)
        return fail(FA_ERR_INDEX_SPACE_EXCEEDED, "paged decode exceeds the i32 index space");
    // Q, O and pool byte sizes (head_dim <= 128 here, so head_dim * 4 cannot overflow)
    if (mul_ov(n_seqs, q_heads, &x) || mul_ov(x, head_dim * 4, &x) ||
        mul_ov(rows, kv_heads, &x) || mul_ov(x, head_dim * 4, &x))
        return fail(FA_ERR_SHAPE_OVERFLOW, "attention shape overflows the address space");
    uint64_t max_pos = 0;
    std::vector<int32_t>& qpos = *qpos_out;
    qpos.resize(n_seqs);
    for (uint64_t s = 0; s < n_seqs; ++s) {
        if (ctx_lens[s] <= 0)
            return fail(FA_ERR_EMPTY_TABLE, "paged decode requires at least one live KV token");
        const int32_t qp = q_positions ? q_positions[s] : ctx_lens[s] - 1;
        if (qp < 0)
            return fail(FA_ERR_POSITION_OVERFLOW, "rotary position offset overflows the index space");
        if (cfg && cfg->causal && (int64_t)qp + 1 < (int64_t)ctx_lens[s])
            return fail(FA_ERR_CAUSAL_VISIBILITY_MISMATCH,
                        "paged causal decode query position %d cannot see all %d live KV tokens",
                        qp, ctx_lens[s]);
        qpos[s] = qp;
        max_pos = std::max<uint64_t>(max_pos, (uint64_t)qp + 1);
    }
    if (int rc = check_pages(block_tables, max_pages, n_seqs, 0, ctx_lens, page_size, physical_pages))
        return rc;
    *max_pos_out = max_pos;
    return FA_OK;
}

}  // namespace

extern "C" {

int fa_paged_decode_prepare(fa_ctx* ctx, const int32_t* block_tables, uint64_t max_pages,
                            const int32_t* ctx_lens, const int32_t* q_positions, uint64_t n_seqs,
                            uint64_t page_size, uint64_t physical_pages, uint64_t q_heads,
                            uint64_t kv_heads, uint64_t head_dim, const fa_config* cfg,
                            float theta, int dtype, fa_decode_plan** out) {
    if (!out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    float scale;
    uint64_t max_pos = 0;
    std::vector<int32_t> qpos;
    if (int rc = validate_decode(block_tables, max_pages, ctx_lens, q_positions, n_seqs, page_size,
                                 physical_pages, q_heads, kv_heads, head_dim, cfg, theta, dtype,
                                 &scale, &qpos, &max_pos))
        return rc;
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    begin_call(ctx);
    if (int rc = set_device(ctx)) return rc;

    fa_decode_plan* p = new fa_decode_plan();
    p->ctx = ctx;
    p->n_seqs = n_seqs;
    p->max_pages = max_pages;
    p->page_size = page_size;
    p->physical_pages = physical_pages;
    p->q_heads = q_heads;
    p->kv_heads = kv_heads;
    p->head_dim = head_dim;
    p->dtype = dtype;
    p->scale = scale;
    p->theta = theta;
    p->ctx_lens.assign(ctx_lens, ctx_lens + n_seqs);
    p->max_pos = max_pos;
    int rc = FA_OK;
    if (!rc) rc = dev_alloc(ctx, (void**)&p->d_bt, n_seqs * max_pages * 4);
    if (!rc) rc = dev_alloc(ctx, (void**)&p->d_ctx, n_seqs * 4);
    if (!rc) rc = dev_alloc(ctx, (void**)&p->d_qpos, n_seqs * 4);
    if (!rc) rc = stage_upload(ctx, p->d_bt, block_tables, n_seqs * max_pages * 4);
    if (!rc) rc = stage_upload(ctx, p->d_ctx, ctx_lens, n_seqs * 4);
    if (!rc) rc = stage_upload(ctx, p->d_qpos, qpos.data(), n_seqs * 4);
    if (!rc) {
        p->split_req = 0;
        rc = build_work(p);
    }
    if (rc) {
        (void)hipStreamSynchronize(ctx->stream);  // error path: no copy may still target it
        free_plan(p);
        return rc;
    }
    *out = p;
    return ok();
}

int fa_paged_decode_plan_set_split(fa_ctx* ctx, fa_decode_plan* p, uint64_t split_tokens) {
    if (!ctx || !p) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (split_tokens % 16)
        return fail(FA_ERR_INDEX_SPACE_EXCEEDED, "split size %llu is not a multiple of 16",
                    (unsigned long long)split_tokens);
    if (split_tokens > max_split_tokens(p->page_size))
        return fail(FA_ERR_INDEX_SPACE_EXCEEDED,
                    "split size %llu spans more than 64 pages of %llu tokens",
                    (unsigned long long)split_tokens, (unsigned long long)p->page_size);
    if (int rc = set_device(ctx)) return rc;
    p->split_req = split_tokens;
    if (int rc = build_work(p)) return rc;
    return ok();
}

int fa_paged_decode_plan_info(const fa_decode_plan* p, uint64_t* split_tokens,
                              uint64_t* work_items, uint64_t* workspace_bytes) {
    if (!p) return fail(FA_ERR_NULL_ARGUMENT, "plan is null");
    if (split_tokens) *split_tokens = p->split_tokens;
    // one work item = one (segment, unit) pair; a head-grouped segment serves every unit
    if (work_items) *work_items = p->grouped > 0 ? p->n_work * p->units : p->n_work;
    if (workspace_bytes) *workspace_bytes = p->part_bytes;
    return ok();
}

int fa_paged_decode_plan_destroy(fa_decode_plan* p) {
    if (!p) return ok();
    if (p->ctx && p->ctx->capturing)
        return refuse_in_capture(p->ctx, "release (it waits for the stream)");
    (void)hipSetDevice(p->ctx->device);
    (void)hipStreamSynchronize(p->ctx->stream);
    free_plan(p);
    return ok();
}

}  // extern "C"

namespace {

// Enqueues the split kernel and the combine of plan `p` (device state in place) with the RoPE
// (cos, sin) rows `table` addressed by the plan's query positions.
int enqueue_decode(fa_ctx* ctx, const fa_decode_plan* p, const float2* table, const void* q,
                   const void* k_pool, const void* v_pool, void* out_lse,
                   const fa_packed_layout& lay) {
    fa::DecodeArgs a{};
    a.q = q;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.o = out_lse;
    a.lse = (float*)((uint8_t*)out_lse + lay.lse_byte_offset);
    a.block_tables = p->d_bt;
    a.ctx_lens = p->d_ctx;
    a.q_positions = p->d_qpos;
    a.seg = p->d_work;
    a.wave_off = p->d_work + 5 * p->n_work;
    a.unit_part = a.wave_off + p->n_waves + 1;
    a.part_o = p->d_part;
    a.part_ml = p->d_part + std::max<uint64_t>(1, p->n_slots) * 16 * p->head_dim;
    if (!a.part_o || !a.block_tables || !a.seg)
        return fail(FA_ERR_NULL_ARGUMENT, "decode plan is missing device state");
    a.rope_table = table;
    a.n_seqs = (int)p->n_seqs;
    a.n_waves = (int)p->n_waves;
    a.chunks = (int)p->units / (int)p->kv_heads;
    a.q_heads = (int)p->q_heads;
    a.kv_heads = (int)p->kv_heads;
    a.group = (int)(p->q_heads / p->kv_heads);
    a.head_dim = (int)p->head_dim;
    a.page_size = (int)p->page_size;
    a.bt_stride = (int)p->max_pages;
    a.scale = p->scale;
    a.grouped = p->grouped;
    unsigned grid[3], block;
    int dispatches = 0;
    bool mfma = false;
    DecodeMarks marks{ctx, &mfma};
    // the head-grouped split kernel records its span's events as part of its dispatch
    if (p->dtype != FA_DTYPE_F32 && p->page_size % 16 == 0 && p->grouped > 0 &&
        dispatch_events(ctx, &a.ev_start, &a.ev_stop)) {
        marks.own = true;
        marks.start = a.ev_start;
        marks.stop = a.ev_stop;
    } else {
        begin_span(ctx);
    }
    fa::launch_decode((Dtype)p->dtype, a, ctx->stream, grid, &block, &dispatches, &mfma,
                      &DecodeMarks::between, &marks);
    end_span(ctx, FA_KERNEL_DECODE_COMBINE);
    HIP_TRY(hipGetLastError());
    const int kid = mfma ? FA_KERNEL_DECODE_PAGED_MFMA : FA_KERNEL_DECODE_PAGED_SPLITK;
    record(ctx, kid,
           mfma && p->grouped ? "decode_mfma_grouped + decode_combine" : kernel_name(kid),
           (uint32_t)std::min<uint64_t>(16, p->q_heads / p->kv_heads), 16, grid, block,
           (uint32_t)dispatches, (uint32_t)((p->split_tokens)), nullptr);
    return FA_OK;
}

// The enqueue half of fa_paged_decode_noalloc, run while the device's scratch is held.
int noalloc_enqueue(fa_ctx* ctx, uint8_t* base, const int32_t* h, uint64_t meta_ints,
                    uint64_t n_bt, uint64_t n_seqs, uint64_t rope_bytes, uint64_t part_bytes,
                    float theta, uint64_t head_dim, fa_decode_plan* pp, const void* q,
                    const void* k_pool, const void* v_pool, void* out_lse,
                    const fa_packed_layout& lay);

}  // namespace

extern "C" {

int fa_paged_decode_launch(fa_ctx* ctx, const fa_decode_plan* p, const void* q, size_t q_bytes,
                           const void* k_pool, const void* v_pool, size_t pool_bytes,
                           void* out_lse, size_t out_bytes) {
    if (!ctx || !p) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    begin_call(ctx);
    const uint64_t eb = elem_bytes(p->dtype);
    const uint64_t qn = p->n_seqs * p->q_heads * p->head_dim;
    const uint64_t pool = p->physical_pages * p->page_size * p->kv_heads * p->head_dim * eb;
    fa_packed_layout lay;
    if (int rc = fa_packed_layout_for(qn, p->n_seqs * p->q_heads, p->dtype, &lay)) return rc;
    if (int rc = check_buffer("Q", q, q_bytes, qn * eb)) return rc;
    if (int rc = check_buffer("K", k_pool, pool_bytes, pool)) return rc;
    if (int rc = check_buffer("V", v_pool, pool_bytes, pool)) return rc;
    if (int rc = check_buffer("O|LSE", out_lse, out_bytes, lay.combined_bytes)) return rc;
    if (int rc = set_device(ctx)) return rc;
    const float2* table = nullptr;
    if (int rc = ensure_rope(ctx, p->theta, p->head_dim, p->max_pos, &table)) return rc;
    if (int rc = enqueue_decode(ctx, p, table, q, k_pool, v_pool, out_lse, lay)) return rc;
    return ok();
}

int fa_paged_decode_noalloc(fa_ctx* ctx, const int32_t* block_tables, uint64_t max_pages,
                            const int32_t* ctx_lens, const int32_t* q_positions, uint64_t n_seqs,
                            uint64_t page_size, uint64_t physical_pages, uint64_t q_heads,
                            uint64_t kv_heads, uint64_t head_dim, const fa_config* cfg,
                            float theta, int dtype, const void* q, size_t q_bytes,
                            const void* k_pool, const void* v_pool, size_t pool_bytes,
                            void* out_lse, size_t out_bytes) {
    float scale;
    uint64_t max_pos = 0;
    std::vector<int32_t> qpos;
    if (int rc = validate_decode(block_tables, max_pages, ctx_lens, q_positions, n_seqs, page_size,
                                 physical_pages, q_heads, kv_heads, head_dim, cfg, theta, dtype,
                                 &scale, &qpos, &max_pos))
        return rc;
    const uint64_t eb = elem_bytes(dtype);
    const uint64_t qn = n_seqs * q_heads * head_dim;
    const uint64_t pool = physical_pages * page_size * kv_heads * head_dim * eb;
    fa_packed_layout lay;
    if (int rc = fa_packed_layout_for(qn, n_seqs * q_heads, dtype, &lay)) return rc;
    if (int rc = check_buffer("Q", q, q_bytes, qn * eb)) return rc;
    if (int rc = check_buffer("K", k_pool, pool_bytes, pool)) return rc;
    if (int rc = check_buffer("V", v_pool, pool_bytes, pool)) return rc;
    if (int rc = check_buffer("O|LSE", out_lse, out_bytes, lay.combined_bytes)) return rc;
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    begin_call(ctx);
    // the metadata is copied from a host staging area that the next call rewrites: a graph
    // replay would read whatever that area holds by then
    if (int rc = refuse_in_capture(ctx, "host upload")) return rc;
    if (int rc = set_device(ctx)) return rc;
    if (!ctx->na_scratch || !ctx->na_copied || !ctx->na_host)
        return fail(FA_ERR_HIP, "the static decode scratch of device %d is not addressable",
                    ctx->device);

    // The plan lives on the stack; its device state points into the scratch.
    fa_decode_plan p;
    p.ctx = ctx;
    p.n_seqs = n_seqs;
    p.max_pages = max_pages;
    p.page_size = page_size;
    p.physical_pages = physical_pages;
    p.q_heads = q_heads;
    p.kv_heads = kv_heads;
    p.head_dim = head_dim;
    p.dtype = dtype;
    p.scale = scale;
    p.theta = theta;
    p.ctx_lens.assign(ctx_lens, ctx_lens + n_seqs);
    p.max_pos = max_pos;
    p.split_req = 0;
    std::vector<int32_t> work;
    if (int rc = compute_work(&p, &work)) return rc;

    // Scratch layout: [metadata (kNoAllocMetaBytes) | (cos, sin) rows of the queries | partials].
    // Metadata ints: block tables | context lengths | query positions | 0..n_seqs-1 (each query's
    // row of the compact table) | work list.
    const uint64_t n_bt = n_seqs * max_pages;
    const uint64_t meta_ints = n_bt + 4 * n_seqs + work.size();
    const uint64_t rope_bytes = (n_seqs * (head_dim / 2) * sizeof(float2) + 255) / 256 * 256;
    const uint64_t part_bytes = partial_bytes(&p);
    if (meta_ints * 4 > kNoAllocMetaBytes)
        return fail(FA_ERR_SCRATCH_EXCEEDED,
                    "allocation-free decode needs %llu bytes of block tables and work lists; "
                    "its scratch holds %llu",
                    (unsigned long long)(meta_ints * 4), (unsigned long long)kNoAllocMetaBytes);
    if (kNoAllocMetaBytes + rope_bytes + part_bytes > fa::kNoAllocScratchBytes)
        return fail(FA_ERR_SCRATCH_EXCEEDED,
                    "allocation-free decode needs %llu bytes of scratch; the static scratch "
                    "holds %llu",
                    (unsigned long long)(kNoAllocMetaBytes + rope_bytes + part_bytes),
                    (unsigned long long)fa::kNoAllocScratchBytes);
    // the previous call's copy must have left the host staging area before it is rewritten
    if (ctx->na_pending) {
        HIP_TRY(hipEventSynchronize(ctx->na_copied));
        ctx->na_pending = false;
    }
    int32_t* h = ctx->na_host;
    memcpy(h, block_tables, n_bt * 4);
    memcpy(h + n_bt, ctx_lens, n_seqs * 4);
    memcpy(h + n_bt + n_seqs, qpos.data(), n_seqs * 4);
    for (uint64_t s = 0; s < n_seqs; ++s) h[n_bt + 2 * n_seqs + s] = (int32_t)s;
    memcpy(h + n_bt + 3 * n_seqs, work.data(), work.size() * 4);
    uint8_t* base = (uint8_t*)ctx->na_scratch;
    // Every context on this device shares the scratch: wait (on the GPU) for the previous
    // user's kernels before overwriting it, and publish this call's completion afterwards.
    if (hipError_t e = fa::noalloc_order_begin(ctx->device, ctx->stream))
        return fail(FA_ERR_HIP, "ordering the shared decode scratch: %s", hipGetErrorString(e));
    const int rc = noalloc_enqueue(ctx, base, h, meta_ints, n_bt, n_seqs, rope_bytes, part_bytes,
                                   theta, head_dim, &p, q, k_pool, v_pool, out_lse, lay);
    const hipError_t e = fa::noalloc_order_end(ctx->device, ctx->stream, true);
    if (rc) return rc;
    if (e != hipSuccess)
        return fail(FA_ERR_HIP, "ordering the shared decode scratch: %s", hipGetErrorString(e));
    return ok();
}

}  // extern "C"

namespace {
int noalloc_enqueue(fa_ctx* ctx, uint8_t* base, const int32_t* h, uint64_t meta_ints,
                    uint64_t n_bt, uint64_t n_seqs, uint64_t rope_bytes, uint64_t part_bytes,
                    float theta, uint64_t head_dim, fa_decode_plan* pp, const void* q,
                    const void* k_pool, const void* v_pool, void* out_lse,
                    const fa_packed_layout& lay) {
    fa_decode_plan& p = *pp;
    HIP_TRY(hipMemcpyAsync(base, h, meta_ints * 4, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipEventRecord(ctx->na_copied, ctx->stream));
    ctx->na_pending = true;
    int32_t* d = (int32_t*)base;
    p.d_bt = d;
    p.d_ctx = d + n_bt;
    const int32_t* d_positions = p.d_ctx + n_seqs;
    p.d_qpos = p.d_ctx + 2 * n_seqs;
    p.d_work = p.d_ctx + 3 * n_seqs;
    float2* table = (float2*)(base + kNoAllocMetaBytes);
    p.d_part = (float*)(base + kNoAllocMetaBytes + rope_bytes);
    p.part_bytes = part_bytes;
    // Nothing in the scratch has to start at zero: every partial slot is written by its segment
    // before the combine reads it.
    begin_span(ctx);
    fa::launch_rope_rows(table, rope_freqs(theta, head_dim), d_positions, (int)n_seqs,
                         (int)(head_dim / 2), ctx->stream);
    end_span(ctx, FA_KERNEL_ROPE_TABLE);
    HIP_TRY(hipGetLastError());
    if (int rc = enqueue_decode(ctx, &p, table, q, k_pool, v_pool, out_lse, lay)) return rc;
    return FA_OK;
}
}  // namespace

extern "C" {

int fa_paged_cache_decode(fa_ctx* ctx, const fa_paged_cache* c, const void* q, size_t q_bytes,
                          uint64_t q_heads, const fa_config* cfg, float theta,
                          uint64_t q_rope_position, void* out_lse, size_t out_bytes) {
    if (!ctx || !c) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    uint64_t mapped = 0;
    if (int rc = fa_kv_table_block_row(&c->table, nullptr, 0, &mapped)) return rc;
    std::vector<int32_t> row(mapped);
    if (int rc = fa_kv_table_block_row(&c->table, row.data(), mapped, &mapped)) return rc;
    if (c->table.live > kI32 || q_rope_position > kI32)
        return fail(FA_ERR_INDEX_SPACE_EXCEEDED, "paged decode exceeds the i32 index space");
    const int32_t len = (int32_t)c->table.live, qp = (int32_t)q_rope_position;
    fa_decode_plan* p = nullptr;
    if (int rc = fa_paged_decode_prepare(ctx, row.data(), mapped, &len, &qp, 1, c->table.page_size,
                                         c->table.physical_pages, q_heads, c->kv_heads,
                                         c->head_dim, cfg, theta, c->dtype, &p))
        return rc;
    const uint32_t allocs = ctx->call_allocs;
    const uint64_t abytes = ctx->call_alloc_bytes;
    int rc = fa_paged_decode_launch(ctx, p, q, q_bytes, c->k, c->v, c->tensor_bytes, out_lse,
                                    out_bytes);
    ctx->last.temporary_allocation_count += allocs;
    ctx->last.temporary_allocation_bytes += abytes;
    fa_paged_decode_plan_destroy(p);
    return rc ? rc : ok();
}

// ---------------------------------------------------------------------------- resident KV
// WgpuResidentKvCache src/wgpu_kv_cache.rs:79: fixed-capacity K and V
// [batch, capacity, kv_heads*head_dim] with one logical length shared by the batch.
struct fa_resident_cache {
    fa_ctx* ctx = nullptr;
    uint64_t batch = 0, kv_heads = 0, capacity = 0, head_dim = 0, row_bytes = 0;
    uint64_t tensor_bytes = 0, len = 0;
    int dtype = 0;
    void* k = nullptr;
    void* v = nullptr;
};

int fa_resident_cache_create(fa_ctx* ctx, uint64_t batch, uint64_t kv_heads, uint64_t capacity,
                             uint64_t head_dim, int dtype, fa_resident_cache** out) {
    if (!ctx || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    if (int rc = check_dtype(dtype)) return rc;
    if (!batch || !kv_heads || !capacity || !head_dim)
        return fail(FA_ERR_ZERO_DIMENSION, "resident KV cache dimensions must be non-zero");
    uint64_t row_el, row_b, rows, bytes;
    if (mul_ov(kv_heads, head_dim, &row_el) || mul_ov(row_el, elem_bytes(dtype), &row_b) ||
        mul_ov(batch, capacity, &rows) || mul_ov(rows, row_b, &bytes))
        return fail(FA_ERR_SHAPE_OVERFLOW, "resident KV cache shape overflows the address space");
    if (int rc = set_device(ctx)) return rc;
    fa_resident_cache* c = new fa_resident_cache();
    c->ctx = ctx;
    c->batch = batch;
    c->kv_heads = kv_heads;
    c->capacity = capacity;
    c->head_dim = head_dim;
    c->row_bytes = row_b;
    c->tensor_bytes = bytes;
    c->dtype = dtype;
    if (hipMalloc(&c->k, bytes) != hipSuccess || hipMalloc(&c->v, bytes) != hipSuccess) {
        if (c->k) (void)hipFree(c->k);
        delete c;
        return fail(FA_ERR_HIP, "resident KV cache requires %llu bytes per tensor",
                    (unsigned long long)bytes);
    }
    *out = c;
    return ok();
}

int fa_resident_cache_destroy(fa_resident_cache* c) {
    if (!c) return ok();
    if (c->ctx && c->ctx->capturing)
        return refuse_in_capture(c->ctx, "release (it waits for the stream)");
    (void)hipSetDevice(c->ctx->device);
    (void)hipStreamSynchronize(c->ctx->stream);
    (void)hipFree(c->k);
    (void)hipFree(c->v);
    delete c;
    return ok();
}

// record_append src/wgpu_kv_cache.rs:212: batch b's source rows [b, append_len) land at cache
// rows b*capacity + len ..; the prefix is never moved; the length advances once every copy of
// the append is enqueued.
int fa_resident_cache_append(fa_resident_cache* c, const void* k_src, const void* v_src,
                             size_t src_bytes, uint64_t append_len, uint64_t* new_len) {
    if (!c) return fail(FA_ERR_NULL_ARGUMENT, "cache is null");
    fa_ctx* ctx = c->ctx;
    begin_call(ctx);
    if (append_len == 0)
        return fail(FA_ERR_ZERO_DIMENSION, "resident KV cache dimensions must be non-zero");
    const uint64_t grown = c->len + append_len;
    if (grown < c->len)
        return fail(FA_ERR_SHAPE_OVERFLOW, "resident KV cache shape overflows the address space");
    if (grown > c->capacity)
        return fail(FA_ERR_CAPACITY_EXCEEDED,
                    "resident KV cache append %llu at length %llu exceeds capacity %llu",
                    (unsigned long long)append_len, (unsigned long long)c->len,
                    (unsigned long long)c->capacity);
    uint64_t per_batch, need;
    if (mul_ov(append_len, c->row_bytes, &per_batch) || mul_ov(c->batch, per_batch, &need))
        return fail(FA_ERR_SHAPE_OVERFLOW, "resident KV cache shape overflows the address space");
    if (int rc = check_buffer("K", k_src, src_bytes, need)) return rc;
    if (int rc = check_buffer("V", v_src, src_bytes, need)) return rc;
    if (int rc = set_device(ctx)) return rc;
    // one strided copy per tensor: batch rows of per_batch bytes, pitches src per_batch,
    // dst capacity*row_bytes
    const size_t dpitch = (size_t)(c->capacity * c->row_bytes);
    uint8_t* kd = (uint8_t*)c->k + c->len * c->row_bytes;
    uint8_t* vd = (uint8_t*)c->v + c->len * c->row_bytes;
    HIP_TRY(hipMemcpy2DAsync(kd, dpitch, k_src, (size_t)per_batch, (size_t)per_batch,
                             (size_t)c->batch, hipMemcpyDeviceToDevice, ctx->stream));
    HIP_TRY(hipMemcpy2DAsync(vd, dpitch, v_src, (size_t)per_batch, (size_t)per_batch,
                             (size_t)c->batch, hipMemcpyDeviceToDevice, ctx->stream));
    c->len = grown;
    if (new_len) *new_len = grown;
    unsigned grid[3] = {(unsigned)append_len, (unsigned)c->batch, 1};
    record(ctx, FA_KERNEL_PAGED_APPEND, "resident append (strided copies)", 0,
           (uint32_t)c->capacity, grid, 0, 2, 1, nullptr);
    return ok();
}

int fa_resident_cache_reset(fa_resident_cache* c) {  // reset :200 (metadata only)
    if (!c) return fail(FA_ERR_NULL_ARGUMENT, "cache is null");
    c->len = 0;
    return ok();
}

uint64_t fa_resident_cache_len(const fa_resident_cache* c) { return c ? c->len : 0; }
void* fa_resident_cache_k(fa_resident_cache* c) { return c ? c->k : nullptr; }
void* fa_resident_cache_v(fa_resident_cache* c) { return c ? c->v : nullptr; }
size_t fa_resident_cache_bytes(const fa_resident_cache* c) { return c ? (size_t)c->tensor_bytes : 0; }

// WgpuResidentDecodePipeline::encode_external_pre_rotated_k src/wgpu_decode.rs:301 (checks in
// the order of validate_external_semantics :419 and validate_kv_view :467). The fixed-capacity
// layout is a page pool with one page of `capacity` rows per batch element, so the plan is a
// paged decode plan whose block table row b is [b].
int fa_resident_decode_prepare(fa_ctx* ctx, uint64_t batch, uint64_t capacity, uint64_t kv_len,
                               uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                               const fa_config* cfg, float theta, uint64_t q_rope_position,
                               int dtype, fa_decode_plan** out) {
    if (!out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    if (cfg && cfg->causal && q_rope_position + 1 < kv_len)
        return fail(FA_ERR_CAUSAL_VISIBILITY_MISMATCH,
                    "resident causal decode query position %llu cannot see all %llu live KV rows",
                    (unsigned long long)q_rope_position, (unsigned long long)kv_len);
    if (!batch || !kv_heads || !capacity || !head_dim)
        return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
    if (kv_len == 0) return fail(FA_ERR_EMPTY_CACHE, "resident decode requires at least one live KV row");
    if (kv_len > capacity)
        return fail(FA_ERR_INVALID_CACHE_LENGTH,
                    "resident decode live KV length %llu exceeds physical capacity %llu",
                    (unsigned long long)kv_len, (unsigned long long)capacity);
    if (batch > kI32 || capacity > kI32 || kv_len > kI32 || q_rope_position > kI32)
        return fail(FA_ERR_INDEX_SPACE_EXCEEDED, "resident decode exceeds the i32 index space");
    std::vector<int32_t> table(batch), lens(batch, (int32_t)kv_len), qpos(batch, (int32_t)q_rope_position);
    for (uint64_t b = 0; b < batch; ++b) table[b] = (int32_t)b;
    return fa_paged_decode_prepare(ctx, table.data(), 1, lens.data(), qpos.data(), batch, capacity,
                                   batch, q_heads, kv_heads, head_dim, cfg, theta, dtype, out);
}

// WgpuResidentDecodePipeline::encode src/wgpu_decode.rs:265: decode over the cache's live rows.
int fa_resident_cache_decode(fa_ctx* ctx, const fa_resident_cache* c, const void* q,
                             size_t q_bytes, uint64_t q_heads, const fa_config* cfg, float theta,
                             uint64_t q_rope_position, void* out_lse, size_t out_bytes) {
    if (!ctx || !c) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    // encode_view :332 checks no causal visibility (the pass carries no causal position);
    // decode attends every live row either way
    fa_config nc{};
    if (cfg) nc = *cfg;
    nc.causal = 0;
    fa_decode_plan* p = nullptr;
    if (int rc = fa_resident_decode_prepare(ctx, c->batch, c->capacity, c->len, q_heads,
                                            c->kv_heads, c->head_dim, &nc, theta,
                                            q_rope_position, c->dtype, &p))
        return rc;
    const uint32_t allocs = ctx->call_allocs;
    const uint64_t abytes = ctx->call_alloc_bytes;
    int rc = fa_paged_decode_launch(ctx, p, q, q_bytes, c->k, c->v, c->tensor_bytes, out_lse,
                                    out_bytes);
    ctx->last.temporary_allocation_count += allocs;
    ctx->last.temporary_allocation_bytes += abytes;
    fa_paged_decode_plan_destroy(p);
    return rc ? rc : ok();
}

// ExternalAsymmetricProjectionRotaryGroupedPipeline::encode_pre_rotated_k_decode_kv_reuse
// src/wgpu_external_asymmetric.rs:216: the candidate's own shape checks, then those of
// encode_with_options :291. The [batch, kv_len, Hkv*D] K/V tensors are a page pool with one
// kv_len-row page per batch element, so the grouped paged decode runs it: one wave group per
// (sequence, KV head) holds each K/V tile once for all q_heads / kv_heads query heads. Causal
// masking at query_position_offset p keeps keys 0..p, i.e. a live length of min(kv_len, p + 1).
// Head dims the decode kernels do not tile (not a multiple of 4 for f32, 8 for 16-bit) take the
// pre-rotated-K prefill kernel, whose result is the same attention.
int fa_forward_projection_asymmetric_decode_kv_reuse(fa_ctx* ctx, const void* q, size_t q_bytes,
                                                     const void* k, const void* v,
                                                     size_t kv_bytes, void* out_lse,
                                                     size_t out_bytes,
                                                     const fa_asymmetric_shape* sh,
                                                     const fa_config* cfg,
                                                     const fa_asymmetric_rotary* rot, int dtype) {
    if (!sh || !rot) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = check_dtype(dtype)) return rc;
    if (int rc = check_asymmetric_shape(sh)) return rc;
    if (sh->query_len != 1)
        return fail(FA_ERR_UNSUPPORTED_CANDIDATE_SHAPE,
                    "external FLAT candidate M48 does not support this shape: query_len must "
                    "equal 1");
    if (sh->q_heads / sh->kv_heads < 2)
        return fail(FA_ERR_UNSUPPORTED_CANDIDATE_SHAPE,
                    "external FLAT candidate M48 does not support this shape: GQA group size "
                    "must be at least 2");
    float scale;
    fa_packed_layout lay;
    if (int rc = check_asymmetric_pass(sh, cfg, rot, dtype, q, q_bytes, k, v, kv_bytes, out_lse,
                                       out_bytes, &scale, &lay))
        return rc;
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    if (sh->head_dim % (dtype == FA_DTYPE_F32 ? 4 : 8))
        return fa_forward_projection_asymmetric(ctx, q, q_bytes, k, v, kv_bytes, out_lse,
                                                out_bytes, sh, cfg, rot, 0, dtype);
    const uint64_t live = cfg && cfg->causal
                              ? std::min<uint64_t>(sh->kv_len, sh->query_position_offset + 1)
                              : sh->kv_len;
    std::vector<int32_t> table(sh->batch), lens(sh->batch, (int32_t)live),
        qpos(sh->batch, (int32_t)rot->query_position_offset);
    for (uint64_t b = 0; b < sh->batch; ++b) table[b] = (int32_t)b;
    fa_config nc{};
    if (cfg) nc = *cfg;
    nc.causal = 0;  // applied above as the live length
    // Each batch element is one page of kv_len rows. The per-token path goes through the
    // allocation-free decode (no plan to allocate, upload into and tear down per token); a shape
    // whose work lists or partials exceed its static scratch takes a one-call plan instead,
    // which allocates and waits for the stream when it is destroyed.
    {
        const int rc = fa_paged_decode_noalloc(
            ctx, table.data(), 1, lens.data(), qpos.data(), sh->batch, sh->kv_len, sh->batch,
            sh->q_heads, sh->kv_heads, sh->head_dim, &nc, rot->theta, dtype, q, q_bytes, k, v,
            kv_bytes, out_lse, out_bytes);
        if (rc != FA_ERR_SCRATCH_EXCEEDED) return rc;
    }
    fa_decode_plan* p = nullptr;
    if (int rc = fa_paged_decode_prepare(ctx, table.data(), 1, lens.data(), qpos.data(), sh->batch,
                                         sh->kv_len, sh->batch, sh->q_heads, sh->kv_heads,
                                         sh->head_dim, &nc, rot->theta, dtype, &p))
        return rc;
    const uint32_t allocs = ctx->call_allocs;
    const uint64_t abytes = ctx->call_alloc_bytes;
    int rc = fa_paged_decode_launch(ctx, p, q, q_bytes, k, v, kv_bytes, out_lse, out_bytes);
    ctx->last.temporary_allocation_count += allocs;
    ctx->last.temporary_allocation_bytes += abytes;
    fa_paged_decode_plan_destroy(p);
    return rc ? rc : ok();
}

}  // extern "C"

// ---------------------------------------------------------------------------- paged prefill
struct fa_prefill_plan {
    fa_ctx* ctx = nullptr;
    fa_asymmetric_shape shape{};
    fa_asymmetric_rotary rot{};
    int causal = 0;
    float scale = 0.0f;
    int dtype = 0;
    uint64_t max_pages = 0, page_size = 0, physical_pages = 0;
    int32_t* d_bt = nullptr;
};

extern "C" {

int fa_chunked_prefill_paged_prepare(fa_ctx* ctx, const int32_t* block_tables, uint64_t max_pages,
                                     uint64_t page_size, uint64_t physical_pages,
                                     const fa_asymmetric_shape* sh, const fa_config* cfg,
                                     const fa_asymmetric_rotary* rot, int dtype,
                                     fa_prefill_plan** out) {
    if (!block_tables || !sh || !rot || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    *out = nullptr;
    if (int rc = check_dtype(dtype)) return rc;
    if (!sh->batch || !sh->q_heads || !sh->kv_heads || !sh->query_len || !sh->kv_len ||
        !sh->head_dim || !max_pages)
        return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
    if (!page_size || !physical_pages)
        return fail(FA_ERR_PAGED_ZERO_DIMENSION, "paged KV dimensions must be non-zero");
    if (int rc = validate_grouped(sh->batch, sh->q_heads, sh->kv_heads,
                                  std::max(sh->query_len, sh->kv_len), sh->head_dim))
        return rc;
    // (written so that a position near the top of the u64 range cannot wrap past the test)
    if (sh->query_len > kI32 || sh->query_position_offset > kI32 - sh->query_len)
        return fail(FA_ERR_POSITION_OVERFLOW, "rotary position offset overflows the index space");
    if (int rc = check_rotary(rot->theta, rot->query_position_offset, sh->head_dim, sh->query_len))
        return rc;
    if (int rc = check_head_dim(sh->head_dim, dtype)) return rc;
    float scale;
    if (int rc = resolve_scale(cfg, sh->head_dim, &scale)) return rc;
    uint64_t rows, x;
    if (mul_ov(page_size, physical_pages, &rows) || rows > kI32 || max_pages > kI32 ||
        mul_ov(sh->batch, max_pages, &x) || x > kI32)
        return fail(FA_ERR_INDEX_SPACE_EXCEEDED, "paged prefill exceeds the i32 index space");
    if (mul_ov(rows, sh->kv_heads, &x) || mul_ov(x, sh->head_dim * 4, &x))
        return fail(FA_ERR_SHAPE_OVERFLOW, "attention shape overflows the address space");
    if (int rc = check_pages(block_tables, max_pages, sh->batch, sh->kv_len, nullptr, page_size,
                             physical_pages))
        return rc;
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    begin_call(ctx);
    if (int rc = set_device(ctx)) return rc;
    fa_prefill_plan* p = new fa_prefill_plan();
    p->ctx = ctx;
    p->shape = *sh;
    p->rot = *rot;
    p->causal = cfg && cfg->causal;
    p->scale = scale;
    p->dtype = dtype;
    p->max_pages = max_pages;
    p->page_size = page_size;
    p->physical_pages = physical_pages;
    int rc = dev_alloc(ctx, (void**)&p->d_bt, sh->batch * max_pages * 4);
    if (!rc) rc = stage_upload(ctx, p->d_bt, block_tables, sh->batch * max_pages * 4);
    if (rc) {
        (void)hipStreamSynchronize(ctx->stream);  // error path: no copy may still target it
        if (p->d_bt) (void)hipFree(p->d_bt);
        delete p;
        return rc;
    }
    *out = p;
    return ok();
}

int fa_prefill_plan_destroy(fa_prefill_plan* p) {
    if (!p) return ok();
    if (p->ctx && p->ctx->capturing)
        return refuse_in_capture(p->ctx, "release (it waits for the stream)");
    (void)hipSetDevice(p->ctx->device);
    (void)hipStreamSynchronize(p->ctx->stream);
    if (p->d_bt) (void)hipFree(p->d_bt);
    delete p;
    return ok();
}

int fa_chunked_prefill_paged_launch(fa_ctx* ctx, const fa_prefill_plan* p, const void* q,
                                    size_t q_bytes, const void* k_pool, const void* v_pool,
                                    size_t pool_bytes, void* out_lse, size_t out_bytes) {
    if (!ctx || !p) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    begin_call(ctx);
    const fa_asymmetric_shape& sh = p->shape;
    const uint64_t eb = elem_bytes(p->dtype);
    const uint64_t qn = sh.batch * sh.query_len * sh.q_heads * sh.head_dim;
    const uint64_t pool = p->physical_pages * p->page_size * sh.kv_heads * sh.head_dim * eb;
    fa_packed_layout lay;
    if (int rc = fa_packed_layout_for(qn, sh.batch * sh.q_heads * sh.query_len, p->dtype, &lay))
        return rc;
    if (int rc = check_buffer("Q", q, q_bytes, qn * eb)) return rc;
    if (int rc = check_buffer("K", k_pool, pool_bytes, pool)) return rc;
    if (int rc = check_buffer("V", v_pool, pool_bytes, pool)) return rc;
    if (int rc = check_buffer("O|LSE", out_lse, out_bytes, lay.combined_bytes)) return rc;
    if (int rc = set_device(ctx)) return rc;
    PrefillJob j{};
    j.dt = (Dtype)p->dtype;
    j.dtype = p->dtype;
    j.paged = true;
    j.rope = true;
    j.theta = p->rot.theta;
    j.max_pos = p->rot.query_position_offset + sh.query_len;
    fa::PrefillArgs& a = j.a;
    const int64_t D = (int64_t)sh.head_dim, QW = (int64_t)sh.q_heads * D,
                  KW = (int64_t)sh.kv_heads * D;
    a.q = q; a.k = k_pool; a.v = v_pool;
    a.o = out_lse;
    a.lse = (float*)((uint8_t*)out_lse + lay.lse_byte_offset);
    a.q_sb = (int64_t)sh.query_len * QW; a.q_sh = D; a.q_ss = QW;
    a.k_sb = 0; a.k_sh = D; a.k_ss = KW;
    a.o_sb = a.q_sb; a.o_sh = a.q_sh; a.o_ss = a.q_ss;
    a.lse_sb = (int64_t)sh.q_heads * sh.query_len; a.lse_sh = (int64_t)sh.query_len;
    a.batch = (int)sh.batch; a.q_heads = (int)sh.q_heads; a.kv_heads = (int)sh.kv_heads;
    a.group = (int)(sh.q_heads / sh.kv_heads);
    a.q_len = (int)sh.query_len; a.kv_len = (int)sh.kv_len; a.head_dim = (int)D;
    a.causal = p->causal;
    a.causal_offset = (int)sh.query_position_offset;
    a.rope_q = 1; a.rope_k = 0;  // K in the pool is stored pre-rotated
    a.q_rope_offset = (int)p->rot.query_position_offset;
    a.kv_rope_offset = 0;
    a.scale = p->scale;
    a.block_tables = p->d_bt;
    a.bt_stride = (int)p->max_pages;
    a.page_size = (int)p->page_size;
    if (int rc = run_prefill(ctx, j)) return rc;
    return ok();
}

int fa_paged_append_batched(fa_ctx* ctx, const int32_t* block_tables, uint64_t max_pages,
                            const int32_t* start_lens, uint64_t n_seqs, uint64_t append_len,
                            uint64_t page_size, uint64_t physical_pages, uint64_t kv_heads,
                            uint64_t head_dim, const void* k_src, const void* v_src,
                            size_t src_bytes, void* k_pool, void* v_pool, size_t pool_bytes,
                            const fa_rotary* rot, int dtype) {
    if (!block_tables || !start_lens) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = check_dtype(dtype)) return rc;
    if (!n_seqs || !append_len || !kv_heads || !head_dim || !max_pages)
        return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
    if (!page_size || !physical_pages)
        return fail(FA_ERR_PAGED_ZERO_DIMENSION, "paged KV dimensions must be non-zero");
    if (head_dim % 8)
        return fail(FA_ERR_UNSUPPORTED_HEAD_DIM, "append needs head_dim %% 8 == 0, got %llu",
                    (unsigned long long)head_dim);
    uint64_t rows, cap_tokens, row, src_need, pool_need, x;
    if (mul_ov(page_size, physical_pages, &rows) || rows > kI32 ||
        mul_ov(max_pages, page_size, &cap_tokens) || cap_tokens > kI32)
        return fail(FA_ERR_INDEX_SPACE_EXCEEDED, "paged append exceeds the i32 index space");
    std::vector<int32_t> ends(n_seqs);
    for (uint64_t s = 0; s < n_seqs; ++s) {
        if (start_lens[s] < 0)
            return fail(FA_ERR_INDEX_SPACE_EXCEEDED, "negative start length for sequence %llu",
                        (unsigned long long)s);
        // start_lens[s] < 2^31 and cap_tokens <= 2^31 - 1: compare without forming a sum that
        // could wrap
        if (append_len > cap_tokens || (uint64_t)start_lens[s] > cap_tokens - append_len)
            return fail(FA_ERR_CAPACITY_EXCEEDED,
                        "paged KV append requires %llu tokens, capacity is %llu",
                        (unsigned long long)((uint64_t)start_lens[s] + std::min(append_len, cap_tokens + 1)),
                        (unsigned long long)cap_tokens);
        ends[s] = (int32_t)((uint64_t)start_lens[s] + append_len);
    }
    if (int rc = check_pages(block_tables, max_pages, n_seqs, 0, ends.data(), page_size,
                             physical_pages))
        return rc;
    // every size product is checked: a wrapped size would pass the buffer checks
    if (mul_ov(kv_heads, head_dim, &x) || mul_ov(x, elem_bytes(dtype), &row) ||
        mul_ov(n_seqs, append_len, &x) || mul_ov(x, row, &src_need) ||
        mul_ov(rows, row, &pool_need))
        return fail(FA_ERR_SHAPE_OVERFLOW, "paged append shape overflows the address space");
    if (int rc = check_buffer("K", k_src, src_bytes, src_need)) return rc;
    if (int rc = check_buffer("V", v_src, src_bytes, src_need)) return rc;
    if (int rc = check_buffer("K pool", k_pool, pool_bytes, pool_need)) return rc;
    if (int rc = check_buffer("V pool", v_pool, pool_bytes, pool_need)) return rc;
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    begin_call(ctx);
    if (int rc = set_device(ctx)) return rc;
    const float2* table = nullptr;
    if (rot) {
        uint64_t maxend = 0;
        for (int32_t e : ends) maxend = std::max<uint64_t>(maxend, (uint64_t)e);
        if (int rc = check_rotary(rot->theta, rot->position_offset, head_dim, maxend)) return rc;
        if (int rc = ensure_rope(ctx, rot->theta, head_dim, rot->position_offset + maxend, &table))
            return rc;
    }
    // block tables and start lengths reach the device by one stream-ordered copy
    std::vector<int32_t> meta(block_tables, block_tables + n_seqs * max_pages);
    meta.insert(meta.end(), start_lens, start_lens + n_seqs);
    const int32_t* d_meta = nullptr;
    if (int rc = upload_meta(ctx, meta.data(), meta.size(), &d_meta)) return rc;
    const int32_t* d_bt = d_meta;
    const int32_t* d_start = d_meta + n_seqs * max_pages;
    fa::AppendArgs a{};
    a.k_src = k_src;
    a.v_src = v_src;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.block_tables = d_bt;
    a.start_lens = d_start;
    a.n_seqs = (int)n_seqs;
    a.append_len = (int)append_len;
    a.bt_stride = (int)max_pages;
    a.page_size = (int)page_size;
    a.kv_heads = (int)kv_heads;
    a.head_dim = (int)head_dim;
    a.rope_table = table;
    a.rope_offset = rot ? (int)rot->position_offset : 0;
    begin_span(ctx);
    fa::launch_append((Dtype)dtype, a, ctx->stream);
    end_span(ctx, FA_KERNEL_PAGED_APPEND);
    HIP_TRY(hipGetLastError());
    unsigned grid[3] = {(unsigned)append_len, (unsigned)n_seqs, 1};
    record(ctx, FA_KERNEL_PAGED_APPEND, "append_kernel", 0, (uint32_t)page_size, grid,
           (unsigned)std::min<uint64_t>(256, std::max<uint64_t>(64, kv_heads * head_dim / 8)), 1, 1,
           nullptr);
    return ok();
}

// ------------------------------------------------------------------ recompute backward
// WgpuGroupedBackwardRecomputePipeline src/wgpu_backward_grouped.rs:181-329.

int fa_backward_grouped_layout(const fa_grouped_shape* sh, int dtype, fa_backward_layout* out) {
    if (!sh || !out) return fail(FA_ERR_NULL_ARGUMENT, "null argument");
    if (int rc = check_dtype(dtype)) return rc;
    // shape.validate() then the checked tensor lengths (src/wgpu_backward_grouped.rs:184-187)
    if (!sh->batch || !sh->q_heads || !sh->kv_heads || !sh->seq_len || !sh->head_dim)
        return fail(FA_ERR_ZERO_DIMENSION, "attention dimensions must all be non-zero");
    if (sh->q_heads % sh->kv_heads)
        return fail(FA_ERR_INVALID_HEAD_GROUPING,
                    "q_heads (%llu) must be exactly divisible by kv_heads (%llu)",
                    (unsigned long long)sh->q_heads, (unsigned long long)sh->kv_heads);
    uint64_t qn, kvn, ln, eb = (uint64_t)elem_bytes(dtype), fwd, grads, t;
    if (mul_ov(sh->batch, sh->q_heads, &ln) || mul_ov(ln, sh->seq_len, &ln) ||
        mul_ov(ln, sh->head_dim, &qn) || mul_ov(sh->batch, sh->kv_heads, &kvn) ||
        mul_ov(kvn, sh->seq_len, &kvn) || mul_ov(kvn, sh->head_dim, &kvn) ||
        mul_ov(qn, 3 * eb, &fwd) || mul_ov(kvn, 2 * eb, &t) || fwd + t < fwd)
        return fail(FA_ERR_SHAPE_OVERFLOW, "backward shape overflows the address space");
    fwd += t;
    if (mul_ov(ln, 4, &t) || fwd + t < fwd || mul_ov(qn, eb, &grads) ||
        mul_ov(kvn, 2 * eb, &t) || grads + t < grads)
        return fail(FA_ERR_SHAPE_OVERFLOW, "backward shape overflows the address space");
    grads += t;
    fwd += ln * 4;
    fa_backward_layout& l = *out;
    l.q_elements = qn;
    l.kv_elements = kvn;
    l.lse_elements = ln;
    l.q_offset = 0;
    l.k_offset = qn * eb;
    l.v_offset = l.k_offset + kvn * eb;
    l.d_out_offset = l.v_offset + kvn * eb;
    l.output_offset = l.d_out_offset + qn * eb;
    l.lse_offset = l.output_offset + qn * eb;
    l.packed_forward_bytes = fwd;
    l.dq_offset = 0;
    l.dk_offset = qn * eb;
    l.dv_offset = l.dk_offset + kvn * eb;
    l.gradient_bytes = grads;
    return ok();
}

int fa_backward_grouped(fa_ctx* ctx, const void* q, const void* k, const void* v,
                        const void* d_out, const void* out, const float* lse, void* dq, void* dk,
                        void* dv, const fa_grouped_shape* sh, const fa_config* cfg, int dtype) {
    fa_backward_layout lay;
    if (int rc = fa_backward_grouped_layout(sh, dtype, &lay)) return rc;
    if (int rc = validate_grouped(sh->batch, sh->q_heads, sh->kv_heads, sh->seq_len, sh->head_dim))
        return rc;
    if (int rc = check_head_dim(sh->head_dim, dtype)) return rc;
    const void* ptrs[] = {q, k, v, d_out, out, lse, dq, dk, dv};
    for (const void* p : ptrs)
        if (!p) return fail(FA_ERR_NULL_ARGUMENT, "backward tensor pointer is null");
    float scale;
    if (int rc = resolve_scale(cfg, sh->head_dim, &scale)) return rc;
    if (!ctx) return fail(FA_ERR_NULL_ARGUMENT, "context is null");
    begin_call(ctx);
    if (int rc = set_device(ctx)) return rc;
    void* delta = nullptr;
    if (int rc = grow(ctx, &ctx->ws_delta, &ctx->ws_delta_bytes, lay.lse_elements * 8, &delta))
        return rc;

    fa::BackwardArgs a{};
    a.q = q; a.k = k; a.v = v; a.dout = d_out; a.o = out; a.lse = lse;
    a.dq = dq; a.dk = dk; a.dv = dv;
    a.ld = (float2*)delta;
    a.batch = (int)sh->batch;
    a.q_heads = (int)sh->q_heads;
    a.kv_heads = (int)sh->kv_heads;
    a.group = (int)(sh->q_heads / sh->kv_heads);
    a.seq = (int)sh->seq_len;
    a.head_dim = (int)sh->head_dim;
    a.causal = cfg && cfg->causal;
    a.scale = scale;
    const uint64_t chunk = 16 / (uint64_t)elem_bytes(dtype);
    bool vec = sh->head_dim % chunk == 0;
    for (const void* p : ptrs) vec = vec && ((uintptr_t)p % 16 == 0);
    a.vec = vec;
    a.dma = vec && sh->seq_len * sh->head_dim * (uint64_t)elem_bytes(dtype) < (1ull << 31);
    // Stored dS: 16-bit storage on the transfer path, 8 KiB per (128-query tile, 32-key block)
    // group of the causal or full square, at most 2 GiB (32-bit buffer offsets); otherwise
    // bwd_dq recomputes S and dP.
    if (ctx->backward_ds_policy != 0 && elem_bytes(dtype) == 2 && a.dma) {
        const unsigned __int128 nb = (sh->seq_len + 31) / 32, nt = (sh->seq_len + 127) / 128;
        const unsigned __int128 gph = a.causal ? 2 * nt * (nt + 1) : nt * nb;
        const unsigned __int128 bytes =
            (unsigned __int128)sh->batch * sh->q_heads * gph * 8192u;
        if (bytes <= (unsigned __int128)INT32_MAX) {
            void* ds = nullptr;
            if (int rc = grow(ctx, &ctx->ws_ds, &ctx->ws_ds_bytes, (size_t)bytes, &ds)) return rc;
            a.ds = ds;
            a.ds_nb = (int)nb;
            a.ds_bytes = (int)bytes;
        }
    }
    a.a64 = ctx->backward_kernel_policy != 0;
    bool a64 = false;
    begin_span(ctx);
    fa::launch_backward((Dtype)dtype, a, ctx->stream, &a64);
    end_span(ctx, FA_KERNEL_BACKWARD_RECOMPUTE);
    HIP_TRY(hipGetLastError());
    const unsigned grid[3] = {(unsigned)(((sh->seq_len + 127) / 128) * sh->batch * sh->kv_heads),
                              1, 1};
    char name[64];
    snprintf(name, sizeof name, "bwd_delta + %s + %s<%s>", a64 ? "bwd_dkdv_a64" : "bwd_dkdv",
             a.ds ? "bwd_dq_ds" : "bwd_dq", dtype_name(dtype));
    record(ctx, FA_KERNEL_BACKWARD_RECOMPUTE, name, 128, 64, grid, 256, 3, 1,
           vec ? nullptr : "unaligned tensors or head_dim off the 16-byte chunk: scalar loads");
    return ok();
}

int fa_backward_grouped_recompute(fa_ctx* ctx, const void* packed_forward, size_t forward_bytes,
                                  void* packed_grads, size_t grads_bytes,
                                  const fa_grouped_shape* sh, const fa_config* cfg, int dtype) {
    fa_backward_layout lay;
    if (int rc = fa_backward_grouped_layout(sh, dtype, &lay)) return rc;
    // validate_buffer order of prepare (src/wgpu_backward_grouped.rs:236-241)
    if (int rc = check_buffer("Q|K|V|dO|O|LSE", packed_forward, forward_bytes,
                              lay.packed_forward_bytes))
        return rc;
    if (int rc = check_buffer("dQ|dK|dV", packed_grads, grads_bytes, lay.gradient_bytes))
        return rc;
    const uint8_t* f = (const uint8_t*)packed_forward;
    uint8_t* gr = (uint8_t*)packed_grads;
    return fa_backward_grouped(ctx, f + lay.q_offset, f + lay.k_offset, f + lay.v_offset,
                               f + lay.d_out_offset, f + lay.output_offset,
                               (const float*)(f + lay.lse_offset), gr + lay.dq_offset,
                               gr + lay.dk_offset, gr + lay.dv_offset, sh, cfg, dtype);
}

int fa_backward_layout_mha(const fa_attention_shape* sh, int dtype, fa_backward_layout* out) {
    if (!sh) return fail(FA_ERR_NULL_ARGUMENT, "shape is null");
    const fa_grouped_shape g{sh->batch, sh->heads, sh->heads, sh->seq_len, sh->head_dim};
    return fa_backward_grouped_layout(&g, dtype, out);
}

int fa_backward_recompute_mha(fa_ctx* ctx, const void* packed_forward, size_t forward_bytes,
                              void* packed_grads, size_t grads_bytes,
                              const fa_attention_shape* sh, const fa_config* cfg, int dtype) {
    if (!sh) return fail(FA_ERR_NULL_ARGUMENT, "shape is null");
    const fa_grouped_shape g{sh->batch, sh->heads, sh->heads, sh->seq_len, sh->head_dim};
    return fa_backward_grouped_recompute(ctx, packed_forward, forward_bytes, packed_grads,
                                         grads_bytes, &g, cfg, dtype);
}

}  // extern "C"
