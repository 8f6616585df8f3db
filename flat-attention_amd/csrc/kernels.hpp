// Kernel argument blocks and host-side launchers shared between the HIP translation units and
// the C-ABI host layer (host.cpp). Launchers assume the host layer already validated shapes,
// buffer sizes and page ids; they only enqueue work on `stream`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

enum class Dtype : int { F32 = 0, F16 = 1, BF16 = 2 };

// Prefill / rectangular attention over contiguous or paged K/V.
// Query row (b, h, t) lives at q + b*q_sb + h*q_sh + t*q_ss (head_dim contiguous); the same
// scheme addresses O with o_* strides and LSE with lse_sb/lse_sh (t contiguous).
// Contiguous K/V row (b, kvh, key): k + b*k_sb + kvh*k_sh + key*k_ss.
// Paged K/V row: k + (block_tables[b*bt_stride + key/page_size]*page_size + key%page_size)*k_ss
//                  + kvh*k_sh.
struct PrefillArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    int64_t q_sb, q_sh, q_ss;
    int64_t k_sb, k_sh, k_ss;
    int64_t o_sb, o_sh, o_ss;
    int64_t lse_sb, lse_sh;
    int batch, q_heads, kv_heads, group;
    int q_len, kv_len, head_dim;
    int causal;
    int causal_offset;   // causal position of query t is causal_offset + t
    int rope_q, rope_k;  // rotate Q / K while loading
    int q_rope_offset, kv_rope_offset;
    const float2* rope_table;  // [rows][head_dim/2] (cos, sin)
    float scale;               // softmax scale
    const int* block_tables;   // paged only
    int bt_stride, page_size;
    // Variable-length batch (contiguous K/V only): 4 ints per batch element — active query
    // rows, active K/V rows, causal position and RoPE position of query row 0 — overriding
    // q_len, kv_len, causal_offset and q_rope_offset; padded query rows get O = 0, LSE = -inf.
    // nullptr: every batch element uses the padded extents.
    const int* var_meta;
    // 16-bit contiguous K rotated on load only: carry the rotated Q and K as 16-bit high part +
    // 16-bit residual and take three MFMAs per score block (f32-level scores).
    int split_qk;
    // Allow the assembly main loop (fa_prefill_a64_bf16) where it applies (prefill_a64_eligible).
    int a64;
    // Rows of rope_table (positions it covers); bounds the assembly kernel's table reads.
    int rope_rows;
    // Precise scores in the assembly kernel (contiguous K/V, K rotated by the pre-pass): the
    // bf16 residual of the rotated K, laid out like `k` (launch_rotate_rows_split); null: off.
    const void* k_lo;
    // Timing events the launch records as part of its own dispatch (the assembly kernel and the
    // f32 kernel; null: none), so that a span brackets the kernel alone, as a profiler's dispatch
    // timestamps do.
    hipEvent_t ev_start, ev_stop;
};

// The assembly prefill (64 query rows per wave, code object loaded per device): bf16, Q rotated
// in the kernel (RoPE), K/V of 128 dims not rotated in the kernel (contiguous, or paged with
// 16-row pages), power-of-two GQA group, no variable-length metadata, 16-byte aligned rows and
// slices addressable with 32-bit offsets, module loaded on the current device.
bool prefill_a64_eligible(Dtype dt, bool paged, const PrefillArgs& a);
// Loads the code object on `device` (current); idempotent. Failure leaves the HIP kernels in use.
hipError_t prefill_a64_load(int device);
void launch_prefill_a64(Dtype dt, const PrefillArgs& a, bool paged, hipStream_t s,
                        unsigned grid[3], unsigned* block);
// Workgroups of its persistent grid: min(query blocks, CUs of the current device).
unsigned prefill_a64_workgroups(const PrefillArgs& a);

void launch_prefill(Dtype dt, bool paged, const PrefillArgs& a, hipStream_t s,
                    unsigned grid[3], unsigned* block);
// The grid, workgroup size and query rows per workgroup launch_prefill uses for `a` (host only).
void prefill_geometry(Dtype dt, bool paged, const PrefillArgs& a, unsigned grid[3],
                      unsigned* block, unsigned* rows);

// Paged q_len=1 decode, split-K over the context of every sequence.
struct DecodeArgs {
    const void* q;        // [n_seqs, q_heads*head_dim]
    const void* k_pool;   // [pages, page_size, kv_heads*head_dim]
    const void* v_pool;
    void* o;              // [n_seqs, q_heads*head_dim] (dtype)
    float* lse;           // [n_seqs, q_heads]
    const int* block_tables;  // [n_seqs, bt_stride]
    const int* ctx_lens;      // [n_seqs]
    const int* q_positions;   // [n_seqs] RoPE position of each query
    // Work: a "unit" is (kv head, chunk of <= 16 query heads of its group), u = kvh*chunks + hc.
    // A segment is a key range [k0, k1) of one (sequence, unit); it writes partial slot `slot`,
    // or O and LSE directly when slot < 0 (the segment covers its whole unit).
    const int* seg;        // [n_seg, 5]: seq, unit, k0, k1, slot
    const int* wave_off;   // [n_waves+1]: wave b runs segments wave_off[b] .. wave_off[b+1]-1
    const int* unit_part;  // [n_seqs*units+1]: slots of (s, u) are unit_part[s*units+u] .. next-1
    float* part_o;         // [slots, 16, head_dim] un-normalised partial O
    float* part_ml;        // [slots, 16, 2] partial (max, sum)
    const float2* rope_table;
    int n_seqs, n_waves, q_heads, kv_heads, group, head_dim, chunks;
    int page_size, bt_stride;
    float scale;
    // > 0: head-grouped MFMA split kernel, workgroups of `grouped` waves (one per unit) sharing
    // one segment list; seg[1] is then the partial-slot stride between units.
    int grouped;
    // Timing events the head-grouped split kernel records as part of its own dispatch (null:
    // none), so that a span brackets that kernel alone.
    hipEvent_t ev_start, ev_stop;
};

// Number of workgroups of the split kernel that launch_decode keeps resident at once for this
// configuration (one-wave workgroups, or `grouped`-wave ones when grouped > 0); the work lists
// are built for exactly this many workgroups or fewer.
int decode_resident_waves(Dtype dt, int head_dim, int group, int page_size, int grouped);

// Launches the split kernel (a.n_waves workgroups) then the combine; `between(user)` (if set) runs on the host between
// the two launches. *mfma tells whether the MFMA split kernel was chosen.
void launch_decode(Dtype dt, const DecodeArgs& a, hipStream_t s, unsigned grid[3],
                   unsigned* block, int* dispatches, bool* mfma, void (*between)(void*),
                   void* user);

// Recompute backward of grouped attention. Q, dO, O, dQ: [batch, q_heads, seq, head_dim];
// K, V, dK, dV: [batch, kv_heads, seq, head_dim]; LSE and delta: [batch, q_heads, seq] f32.
// `ld` is scratch of batch*q_heads*seq float2 (LSE * log2 e, rowsum of dO * O), written by the
// first launch. vec: head_dim is a multiple of the 16-byte chunk and every tensor 16-byte
// aligned; dma: vec, and one (batch, head) slice spans less than 2 GiB (32-bit buffer offsets).
struct BackwardArgs {
    const void* q;
    const void* k;
    const void* v;
    const void* dout;
    const void* o;
    const float* lse;
    void* dq;
    void* dk;
    void* dv;
    float2* ld;
    // Stored dS (16-bit storage with DMA only; null: bwd_dq recomputes S and dP). Per (batch,
    // query head) and 128-query tile t, one 8 KiB group per 32-key block kb (kb < 4 t + 4 under a
    // causal mask, else kb < ds_nb = ceil(seq / 32)): group t * ds_nb + kb, or 2 t (t + 1) + kb
    // causal, of the head's 2 nt (nt + 1) (causal) or nt * ds_nb groups, nt = ceil(seq / 128).
    // A group holds the four 32 x 32 blocks of its 32-query rows, 2 KiB each; inside a block,
    // element (q, k) sits at byte 1024 (q >> 4) + 512 ((q >> 3) & 1) + 16 k + 2 (q & 7): the dK
    // product's dS^T fragment (one key, eight consecutive queries per lane) is one 16-byte
    // piece per lane at 1024 h + 16 lane, 1 KiB per store instruction.
    void* ds;
    int ds_nb, ds_bytes;
    int batch, q_heads, kv_heads, group, seq, head_dim, causal, vec, dma;
    float scale;
    // Allow the assembly dK/dV kernel (fa_bwd_dkdv_a64_bf16 / _f16) where bwd_a64_eligible() holds.
    // It reads `ld` as two f32 arrays of batch*q_heads*seq rows, -LSE / scale then -delta.
    int a64;
};
// Three launches: delta, dK/dV (which also writes dS when `ds` is set), dQ. *a64_out (if set)
// tells whether the assembly dK/dV kernel ran.
void launch_backward(Dtype dt, const BackwardArgs& a, hipStream_t s, bool* a64_out = nullptr);

// The assembly dK/dV kernel (gen_bwd_a64.py): bf16 or f16, head_dim 128, seq a multiple of 128, dS
// stored, 16-byte aligned tensors, 32-bit offsets; its module loaded on the current device.
bool bwd_a64_eligible(Dtype dt, const BackwardArgs& a);
hipError_t bwd_a64_load(int device);
void launch_bwd_a64(Dtype dt, const BackwardArgs& a, hipStream_t s);

// (cos, sin) table: table[pos*half + p] for pos < rows, p < half = head_dim/2, with
// angle = float(pos) * inv_freq[p]. The frequencies travel in the kernel arguments (no copy).
struct RopeFreqs {
    float inv_freq[64];
};
void launch_rope_table(float2* table, const RopeFreqs& f, int rows, int half, hipStream_t s);
// (cos, sin) rows of n listed positions: table[i*half + p] for position positions[i], with the
// same angle expression as launch_rope_table (bitwise equal rows).
void launch_rope_rows(float2* table, const RopeFreqs& f, const int* positions, int n, int half,
                      hipStream_t s);

// Allocation-free paged decode: size of the per-device static scratch array and its device
// address (resolved once per device with hipGetSymbolAddress; never the array's host-side name).
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
hipError_t noalloc_scratch(int device, void** out);
// Orders every use of a device's scratch across streams and contexts: begin locks the device's
// mutex and makes `s` wait (on the GPU) for the previous user's completion event; end records
// this call's completion into that event (when it enqueued work) and unlocks. Every begin that
// returns hipSuccess is paired with one end.
hipError_t noalloc_order_begin(int device, hipStream_t s);
hipError_t noalloc_order_end(int device, hipStream_t s, bool enqueued);

// Scatter `append_len` rows per sequence into the page pool, optionally rotating K rows.
struct AppendArgs {
    const void* k_src;   // [n_seqs, append_len, kv_heads*head_dim]
    const void* v_src;
    void* k_pool;
    void* v_pool;
    const int* block_tables;
    const int* start_lens;   // device [n_seqs], or null with start_len_const
    int start_len_const;
    int n_seqs, append_len, bt_stride, page_size, kv_heads, head_dim;
    const float2* rope_table;  // null: copy K as is
    int rope_offset;
};
void launch_append(Dtype dt, const AppendArgs& a, hipStream_t s);

// Rotate every row of a [rows, heads*head_dim] tensor (in place allowed); row r is at RoPE
// position offset + r % period. head_dim must be a multiple of 8.
// bf16 rows rotated as launch_rotate_rows, written as the rounding `hi` and the bf16 rounding of
// the residual `lo` (same layout).
void launch_rotate_rows_split(const void* in, void* hi, void* lo, int rows, int heads,
                              int head_dim, int64_t period, const float2* table, int offset,
                              hipStream_t s);
void launch_rotate_rows(Dtype dt, const void* in, void* out, int rows, int heads, int head_dim,
                        int64_t period, const float2* table, int offset, hipStream_t s);

}  // namespace fa
