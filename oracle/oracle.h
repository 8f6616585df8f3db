/*
 * CPU oracle for the FLAT-ATTENTION hot path — TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the reference crate's scalar Rust oracles. Only tests/, the smoke
 * check in __graft_entry__.py and bench.py's cpu_baseline leg may load it, and only as the
 * checker or as the timed CPU baseline. The product library never links or calls it.
 *
 * Loop order, operation order and libm calls follow the reference (cited per function) and the
 * file is compiled with -ffp-contract=off so no multiply-add is fused, as in Rust.
 *
 * Every function returns 0 on success or a non-zero fa_status code (include/flat_hip.h).
 * `unit_begin`/`unit_end` restrict the outer (batch, head) loop to units [begin, end) of the
 * flattened batch*heads index (used to time a bounded slice); `threads` > 1 splits the units
 * over POSIX threads (the multi-threaded CPU baseline). Pass 0, UINT64_MAX, 1 for the plain
 * single-threaded reference behaviour.
 */
#ifndef FLAT_ORACLE_H
#define FLAT_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* FlatAttentionConfig::resolved_scale src/lib.rs:257 */
int ora_resolved_scale(int has_scale, float scale, uint64_t head_dim, float* out);

/* forward_reference src/lib.rs:454-520 (MHA, [B,H,S,D]) */
int ora_forward(const float* q, const float* k, const float* v, uint64_t batch, uint64_t heads,
                uint64_t seq, uint64_t dim, int causal, float scale, float* out, float* lse,
                uint64_t unit_begin, uint64_t unit_end, int threads);

/* forward_reference_grouped src/grouped.rs:81-153 */
int ora_forward_grouped(const float* q, const float* k, const float* v, uint64_t batch,
                        uint64_t q_heads, uint64_t kv_heads, uint64_t seq, uint64_t dim,
                        int causal, float scale, float* out, float* lse, uint64_t unit_begin,
                        uint64_t unit_end, int threads);

/* forward_reference_grouped_rope src/rotary_grouped.rs:57-155 */
int ora_forward_grouped_rope(const float* q, const float* k, const float* v, uint64_t batch,
                             uint64_t q_heads, uint64_t kv_heads, uint64_t seq, uint64_t dim,
                             int causal, float scale, float theta, uint64_t position_offset,
                             float* out, float* lse, uint64_t unit_begin, uint64_t unit_end,
                             int threads);

/* forward_reference_projection_grouped_rope_asymmetric src/projection_asymmetric.rs:97-238.
 * rotate_k = 0 treats K as already rotated (the pre-rotated-K contract of the paged cache,
 * shaders/flat_fwd_projection_rope_asymmetric.wgsl:10-12). use_rope = 0 skips RoPE entirely
 * (src/asymmetric_grouped.rs forward_reference_grouped_asymmetric :230 in projection layout). */
int ora_forward_projection_asymmetric(const float* q, const float* k, const float* v,
                                      uint64_t batch, uint64_t q_heads, uint64_t kv_heads,
                                      uint64_t query_len, uint64_t kv_len, uint64_t dim,
                                      uint64_t query_position_offset, int causal, float scale,
                                      int use_rope, float theta, uint64_t q_rope_offset,
                                      uint64_t kv_rope_offset, int rotate_k, float* out,
                                      float* lse, uint64_t unit_begin, uint64_t unit_end,
                                      int threads);

/* forward_reference_projection_grouped_rope_chunked_prefill
 * src/chunked_projection_prefill.rs:63-169 */
int ora_chunked_prefill(const float* q, const float* k, const float* v, uint64_t batch,
                        uint64_t q_heads, uint64_t kv_heads, uint64_t seq, uint64_t dim,
                        int causal, float scale, float theta, uint64_t position_offset,
                        uint64_t query_chunk_size, float* out, float* lse);

/* rotated_pair src/rotary_grouped.rs:37-50 applied to every row of a [rows, heads*dim]
 * projection-layout tensor at position position_offset + row (the rotate_k_projection helper
 * of tests/m16_paged_decode.rs). `positions` != NULL overrides the per-row position. */
int ora_rope_rotate_rows(const float* in, float* out, uint64_t rows, uint64_t heads,
                         uint64_t dim, float theta, uint64_t position_offset,
                         const int64_t* positions);

/* Paged q_len = 1 decode over a shared page pool: gathers each sequence's rows with
 * physical_row = block_table[key / page_size] * page_size + key % page_size
 * (shaders/flat_decode_paged.wgsl:137-154) and runs the asymmetric oracle with query_len 1,
 * kv_len ctx_len, causal offset q_position, pre-rotated K, Q rotated at q_position
 * (tests/m16_paged_decode.rs:171-247). Pool layout [pages, page_size, kv_heads*dim], f32. */
int ora_paged_decode(const float* q, const float* k_pool, const float* v_pool,
                     uint64_t physical_pages, uint64_t page_size, const int32_t* block_tables,
                     uint64_t max_pages, const int32_t* ctx_lens, const int32_t* q_positions,
                     uint64_t n_seqs, uint64_t q_heads, uint64_t kv_heads, uint64_t dim,
                     int causal, float scale, float theta, float* out, float* lse,
                     uint64_t seq_begin, uint64_t seq_end, int threads);

/* Chunked prefill over the page pool (query chunk of query_len rows per sequence at causal
 * offset query_position_offset over kv_len live tokens, pre-rotated K). Gathers and runs the
 * asymmetric oracle per sequence. Q/O projection layout [n_seqs, query_len, q_heads*dim]. */
int ora_paged_prefill(const float* q, const float* k_pool, const float* v_pool,
                      uint64_t physical_pages, uint64_t page_size, const int32_t* block_tables,
                      uint64_t max_pages, uint64_t n_seqs, uint64_t q_heads, uint64_t kv_heads,
                      uint64_t query_len, uint64_t kv_len, uint64_t dim,
                      uint64_t query_position_offset, int causal, float scale, float theta,
                      uint64_t q_rope_offset, float* out, float* lse, uint64_t seq_begin,
                      uint64_t seq_end, int threads);

/* IEEE binary16 round-to-nearest-even: F16::from_f32 / to_f32 src/f16.rs:26-109.
 * bfloat16 follows the same rounding convention on the top 16 bits of binary32. */
uint16_t ora_f32_to_f16(float x);
float ora_f16_to_f32(uint16_t h);
uint16_t ora_f32_to_bf16(float x);
float ora_bf16_to_f32(uint16_t h);
void ora_f32_to_bf16_array(const float* in, uint16_t* out, uint64_t n);
void ora_bf16_to_f32_array(const uint16_t* in, float* out, uint64_t n);
void ora_f32_to_f16_array(const float* in, uint16_t* out, uint64_t n);
void ora_f16_to_f32_array(const uint16_t* in, float* out, uint64_t n);

/* Seeded synthetic input: PCG-style LCG (multiplier 6364136223846793005, increment
 * 1442695040888963407, tests/m38_property_stress.rs:7-30) driving Box-Muller N(0,1) in f32. */
void ora_fill_normal(float* out, uint64_t n, uint64_t seed);

/* backward_reference_grouped src/backward_grouped.rs:17-95: dQ, dK, dV recomputed from
 * Q, K, V, dO and the forward's O and LSE ([B,H,S,D] / [B,Hkv,S,D] / [B,H,S]). Threads split
 * the (batch, kv head) units; each unit keeps the reference's accumulation order. */
int ora_backward_grouped(const float* q, const float* k, const float* v, const float* d_out,
                         const float* out, const float* lse, uint64_t batch, uint64_t q_heads,
                         uint64_t kv_heads, uint64_t seq, uint64_t dim, int causal, float scale,
                         float* dq, float* dk, float* dv, int threads);

#ifdef __cplusplus
}
#endif
#endif
