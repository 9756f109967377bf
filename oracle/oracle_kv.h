/*
 * oracle_kv.h — scalar CPU restatement of AtomFlow's KV-cache hot path.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load liboracle_kv.so, and only as the checker (or as the
 * timed CPU baseline). The product (libatomflow_kv.so) never links or calls it.
 *
 * Each function cites the reference file:line it restates (paths relative to
 * the Altersieg/AtomFlow tree). fp16 is carried as uint16_t bit patterns and
 * converted by hand (IEEE binary16, round-to-nearest-even).
 *
 * Pinning status (what fixes each function besides its own restatement):
 *   ok_f32_to_f16 / ok_f16_to_f32  exhaustive half round trip + ties vs numpy
 *   ok_rope_table                  s=0 closed form, double-precision cos/sin
 *   ok_rope / ok_rope_append       pos 0 identity, pair norm, composition
 *   ok_write_kv_cache              byte copy + untouched canary rows
 *   ok_cached_attention            L=1 -> V, equal keys -> mean(V), dominant
 *                                  key, permutation invariance, torch SDPA (fp64)
 *   ok_e4m3_encode / decode        exhaustive vs torch.float8_e4m3fn
 *   ok_paged_gather                contiguous identity table, permuted tables
 *   ok_w8a16_gemv                  identity weights -> x, power-of-two group
 *   ok_prefill_attention           row i == ok_cached_attention over p0+i+1
 *                                  rows; seq_kv 1 -> V row 0; torch sdpa
 *                                  (causal mask) in float64
 *   ok_prefill_rope_append         == ok_rope_append row by row
 *                                  scales (exact sums), float64 matmul bound
 * The reference ships no golden vectors for this path (its ground_truth *.bin files
 * are full-model activations at seq_len 1).
 */
#ifndef ORACLE_KV_H_
#define ORACLE_KV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint16_t ok_f32_to_f16(float f);
float ok_f16_to_f32(uint16_t h);
void ok_f32_to_f16_array(const float* src, uint16_t* dst, size_t n);
void ok_f16_to_f32_array(const uint16_t* src, float* dst, size_t n);

/* src/kernel/helpers.cu:94-113 */
void ok_rope_table(float* cos_out, float* sin_out, int max_seq, int head_dim, float base);

/* src/kernel/rope.cu:11-46 (token p uses table row p of cos/sin) */
void ok_rope(uint16_t* q, uint16_t* k, const float* cos_cache, const float* sin_cache,
             int seq_len, int kv_head_num, int q_head_num, int head_dim);

/* src/kernel/helpers.cu:126-139 */
void ok_write_kv_cache(const uint16_t* qkv_out, uint16_t* k_cache, uint16_t* v_cache,
                       int current_pos, int q_dim, int kv_dim);

/* src/core/engine.cu:326-355 (rope at table row pos, then write row pos) */
void ok_rope_append(uint16_t* qkv_out, uint16_t* k_cache, uint16_t* v_cache,
                    const float* cos_table, const float* sin_table, int pos, int n_q_heads,
                    int n_kv_heads, int head_dim);

/* src/kernel/tiled_attention.cu:196-269, K/V rows of n_kv_heads*head_dim. */
void ok_cached_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                         uint16_t* out, int seq_len, int head_dim, int n_q_heads, int n_kv_heads);
/* Same computation in double precision, unrounded output (pinning aid). */
void ok_cached_attention_f64(const uint16_t* q, const uint16_t* k_cache,
                             const uint16_t* v_cache, double* out, int seq_len, int head_dim,
                             int n_q_heads, int n_kv_heads);
/* Causal prefill attention, src/kernel/tiled_attention.cu:34-130, generalised to
 * a chunk at cache position p0: query row i (q + i*q_stride) attends cache rows
 * [0, min(p0 + i + 1, kv_len)); output row i at out + i*out_stride. p0 = 0 and
 * kv_len = seq_kv is the reference kernel. Threads split the query rows. */
void ok_prefill_attention(const uint16_t* q, int q_stride, const uint16_t* k_cache,
                          const uint16_t* v_cache, uint16_t* out, int out_stride, int p0, int n,
                          int kv_len, int head_dim, int n_q_heads, int n_kv_heads, int n_threads);
/* Same in double precision, unrounded output [n, n_q_heads*head_dim]. */
void ok_prefill_attention_f64(const uint16_t* q, int q_stride, const uint16_t* k_cache,
                              const uint16_t* v_cache, double* out, int p0, int n, int kv_len,
                              int head_dim, int n_q_heads, int n_kv_heads);
/* n rows of qkv_out (row stride (n_q_heads+2*n_kv_heads)*head_dim): ok_rope_append
 * of row i at position p0 + i (engine.cu:326-355 once per prompt token). */
void ok_prefill_rope_append(uint16_t* qkv_out, int n, uint16_t* k_cache, uint16_t* v_cache,
                            const float* cos_table, const float* sin_table, int p0,
                            int n_q_heads, int n_kv_heads, int head_dim);

/* Multi-threaded form of ok_cached_attention (threads over q heads): the CPU baseline. */
void ok_cached_attention_mt(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                            uint16_t* out, int seq_len, int head_dim, int n_q_heads,
                            int n_kv_heads, int n_threads);

/* FP8 E4M3 (OCP e4m3fn: bias 7, max 448, 0x7F/0xFF NaN). Encode rounds to
 * nearest even after clamping to +-448 (tools/quantize_weights.py:249-260). */
float ok_e4m3_decode(uint8_t code);
uint8_t ok_e4m3_encode(float x);
/* q = encode(clamp(x / scale)) for fp16 inputs. */
void ok_fp8_quantize_f16(const uint16_t* src, uint8_t* dst, size_t n, float scale);

/* Paged pool, one layer slab [total_blocks][block_size][kv_dim] of elem_bytes. */
void ok_paged_gather(const void* slab, const int32_t* block_table, int seq_len, int block_size,
                     int kv_dim, int elem_bytes, void* dst);
/* Paged attention for one sequence: gather + ok_cached_attention (fp16 pool). */
void ok_paged_attention_f16(const uint16_t* q, const uint16_t* k_slab, const uint16_t* v_slab,
                            const int32_t* block_table, int seq_len, int block_size,
                            uint16_t* out, int head_dim, int n_q_heads, int n_kv_heads);
/* Paged attention over an FP8 pool: K/V element = decode(code) * scale[kv_head]. */
void ok_paged_attention_fp8(const uint16_t* q, const uint8_t* k_slab, const uint8_t* v_slab,
                            const float* k_scales, const float* v_scales,
                            const int32_t* block_table, int seq_len, int block_size,
                            uint16_t* out, int head_dim, int n_q_heads, int n_kv_heads);

/* Paged append of one token row (K rotated already): copies K/V (fp16) or
 * quantises them (fp8) into physical row `slot` of the layer slabs. */
void ok_paged_write_f16(const uint16_t* k_row, const uint16_t* v_row, uint16_t* k_slab,
                        uint16_t* v_slab, int64_t slot, int kv_dim);
void ok_paged_write_fp8(const uint16_t* k_row, const uint16_t* v_row, uint8_t* k_slab,
                        uint8_t* v_slab, int64_t slot, int kv_dim, int head_dim,
                        const float* k_scales, const float* v_scales);

/* W8A16 GEMV: y[n] = sum_k e4m3(w[n,k]) * scale[n, k/group_size] * x[k], fp32,
 * rounded to fp16 (src/kernel/qkv_gemm.cu:32-110), in the reference kernel's
 * summation order. w: [n, k] E4M3 codes, x: [k] fp16, scales: [n, k/group_size]
 * fp16, y: [n] fp16. */
void ok_w8a16_gemv(const uint8_t* w, const uint16_t* x, const uint16_t* scales, uint16_t* y,
                   int n, int k, int group_size);
/* Same products summed in double (order-free reference for tolerances). */
void ok_w8a16_gemv_f64(const uint8_t* w, const uint16_t* x, const uint16_t* scales, double* y,
                       int n, int k, int group_size);

#ifdef __cplusplus
}
#endif
#endif
