#pragma once
// C++ operator boundary of the KV-cache hot path: the reference's launcher
// names and argument orders (include/ops/kernel.h:32-42, 93-103, 167-174,
// 195-197) with hipStream_t, plus the fused and paged launchers this build adds.
// Failures throw std::runtime_error carrying the af_kv.h status text (the
// reference aborts in Debug and ignores errors in Release, utils.h:41-118).
// All launchers are asynchronous and safe inside stream capture (except
// build_rope_cache, which copies synchronously, as it runs once at init).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "af_kv.h"
#include "core/view.h"

// kernel.h:32-42 — q [seq_len, q_head_num*head_dim], k [seq_len, kv_head_num*head_dim]
// rotated in place; cos/sin point at the first token's table row.
void launch_rope(const View& q_input, const View& k_input, const float* cos_cache,
                 const float* sin_cache, int seq_len, int kv_head_num, int q_head_num,
                 int head_dim, hipStream_t stream);

// kernel.h:93-103 — seq_len = current_pos + 1 tokens of the [MAX_SEQ_LEN, kv_dim] caches.
void launch_cached_attention(const __half* q, const __half* k_cache, const __half* v_cache,
                             __half* out, int seq_len, int head_dim, int n_q_heads,
                             int n_kv_heads, hipStream_t stream);

// kernel.h:167-174 — row current_pos of the caches from qkv_out [Q | K | V].
// k_cache.dims[0] (MAX_SEQ_LEN) bounds current_pos.
void launch_write_kv_cache(const View& qkv_out, View& k_cache, View& v_cache, int current_pos,
                           int q_dim, int kv_dim, hipStream_t stream);

// kernel.h:195-197 — [max_seq, head_dim/2] fp32 tables, host-computed, copied.
void build_rope_cache(float* d_cos, float* d_sin, int max_seq, int head_dim, float base,
                      hipStream_t stream);

// W8A16 GEMV (kernel.h:138-145 of the reference): FP16 act_x [1, K], FP8
// weight [N, K], FP16 scales [N, K/GS], FP16 output [1, N].
void launch_w8a16_gemv(const View& act_x, const View& weight, const View& scales, View& output,
                       int group_size, hipStream_t stream);

// Legacy causal GQA attention (kernel.h:73-85 of the reference, tiled_attention.cu:
// 136-161): q [seq_q, n_q_heads*head_dim], k/v [seq_kv, n_kv_heads*head_dim];
// query i attends keys s <= i, s < seq_kv. Instantiated for __half.
template <typename T>
void launch_tiled_attention_kernel(const T* q_base, const T* k_base, const T* v_base, T* out,
                                   int seq_q, int seq_kv, int head_dim, int n_q_heads,
                                   int n_kv_heads, hipStream_t stream);

// ---- added by this build ---------------------------------------------------
// Prefill of a prompt chunk: RoPE of qkv_out's n rows at positions p0.. and their
// K/V written to cache rows p0.. (launch_rope with seq_len = n, then
// launch_write_kv_cache per token).
void launch_prefill_rope_append(View& qkv_out, int n, View& k_cache, View& v_cache,
                                const float* cos_table, const float* sin_table, int p0,
                                int n_q_heads, int n_kv_heads, int head_dim, hipStream_t stream);

// Causal attention of a chunk over one sequence's rows of a paged pool (block table
// d_block_table, device int32 [max_blocks]).
void launch_paged_prefill_attention(const __half* q, int q_stride, const af_kv_pool& pool,
                                    int layer, const int32_t* d_block_table, int max_blocks,
                                    int p0, int n, int kv_len, __half* out, int out_stride,
                                    int n_q_heads, hipStream_t stream);

// Causal attention of the chunk's n queries (row stride q_stride) over cache rows
// [0, min(p0 + i + 1, kv_len)) into out (row stride out_stride). head_dim 128.
void launch_prefill_attention(const __half* q, int q_stride, const View& k_cache,
                              const View& v_cache, __half* out, int out_stride, int p0, int n,
                              int kv_len, int n_q_heads, int n_kv_heads, int head_dim,
                              hipStream_t stream);

// The two prefill attention launchers with key pieces (af_prefill_attention_ws,
// af_paged_prefill_attention_ws): a chunk too small to fill the device has its
// heavy query tiles cut into key ranges merged in the kernel. key_pieces 0 =
// the library's choice; workspace of af_prefill_workspace_size bytes, zeroed
// once with af_attention_workspace_init.
void launch_prefill_attention_ws(const __half* q, int q_stride, const View& k_cache,
                                 const View& v_cache, __half* out, int out_stride, int p0, int n,
                                 int kv_len, int n_q_heads, int n_kv_heads, int head_dim,
                                 int key_pieces, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream);
void launch_paged_prefill_attention_ws(const __half* q, int q_stride, const af_kv_pool& pool,
                                       int layer, const int32_t* d_block_table, int max_blocks,
                                       int p0, int n, int kv_len, __half* out, int out_stride,
                                       int n_q_heads, int key_pieces, void* workspace,
                                       size_t workspace_bytes, hipStream_t stream);

// Decode QKV projection + RoPE + KV append (launch_w8a16_gemv, launch_rope and
// launch_write_kv_cache at position pos in one kernel; d_pos overrides pos).
void launch_qkv_rope_append(const View& act_x, const View& w_qkv, const View& scales,
                            int group_size, View& qkv_out, View& k_cache, View& v_cache,
                            const float* cos_table, const float* sin_table, int pos,
                            const int32_t* d_pos, int n_q_heads, int n_kv_heads, int head_dim,
                            hipStream_t stream);

// launch_rope(pos) + launch_write_kv_cache(pos) in one kernel. d_pos (device,
// nullable) overrides pos so a captured graph can advance the position.
void launch_rope_append(View& qkv_out, View& k_cache, View& v_cache, const float* cos_table,
                        const float* sin_table, int pos, const int32_t* d_pos, int n_q_heads,
                        int n_kv_heads, int head_dim, hipStream_t stream);

// Split-K attention with a caller workspace (af_attention_workspace_size) and a
// device-resident length (nullable).
void launch_cached_attention_ws(const __half* q, const __half* k_cache, const __half* v_cache,
                                __half* out, int seq_len, const int32_t* d_seq_len,
                                int max_seq_len, int head_dim, int n_q_heads, int n_kv_heads,
                                int num_splits, void* workspace, size_t workspace_bytes,
                                hipStream_t stream);

void launch_paged_rope_append(__half* qkv_out, int batch, const af_kv_pool& pool, int layer,
                              const int64_t* d_slots, const int32_t* d_positions,
                              const float* cos_table, const float* sin_table, int max_pos,
                              int n_q_heads, hipStream_t stream);

void launch_paged_attention(const __half* q, int q_stride, const af_kv_pool& pool, int layer,
                            const int32_t* d_block_tables, int max_blocks_per_seq,
                            const int32_t* d_seq_lens, int batch, int max_seq_len, __half* out,
                            int out_stride, int n_q_heads, int num_splits, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

void launch_kv_copy_blocks(const af_kv_pool& pool, const int32_t* d_copies, const int32_t* d_count,
                           int max_copies, hipStream_t stream);

// af_paged_decode_fused: paged RoPE + append + attention (lengths = positions + 1).
void launch_paged_decode_fused(__half* qkv_out, int batch, const af_kv_pool& pool, int layer,
                               const int64_t* d_slots, const int32_t* d_positions,
                               const float* cos_table, const float* sin_table, int max_pos,
                               const int32_t* d_block_tables, int max_blocks_per_seq,
                               int max_seq_len, __half* out, int out_stride, int n_q_heads,
                               int num_splits, void* workspace, size_t workspace_bytes,
                               hipStream_t stream);

// af_paged_attention_shared_prefix: forks of one prompt; rows [0, prefix_len)
// through d_prefix_table once for the batch, the rest per sequence.
void launch_paged_attention_shared_prefix(const __half* q, int q_stride, const af_kv_pool& pool,
                                          int layer, const int32_t* d_prefix_table,
                                          int prefix_len, int prefix_splits,
                                          const int32_t* d_block_tables, int max_blocks_per_seq,
                                          const int32_t* d_seq_lens, int batch, int max_seq_len,
                                          __half* out, int out_stride, int n_q_heads,
                                          int num_splits, void* workspace, size_t workspace_bytes,
                                          hipStream_t stream);

// af_paged_decode_fused_shared_prefix: the fused step of a shared-prefix batch.
void launch_paged_decode_fused_shared_prefix(
    __half* qkv_out, int batch, const af_kv_pool& pool, int layer, const int64_t* d_slots,
    const int32_t* d_positions, const float* cos_table, const float* sin_table, int max_pos,
    const int32_t* d_prefix_table, int prefix_len, int prefix_splits,
    const int32_t* d_block_tables, int max_blocks_per_seq, int max_seq_len, __half* out,
    int out_stride, int n_q_heads, int num_splits, void* workspace, size_t workspace_bytes,
    hipStream_t stream);

// W8A16 projections beside the path: the MLP's gate and up GEMVs in one launch
// (engine.cu:418-436 issues two launch_w8a16_gemv), the batched projection of m
// tokens, and the paged serving step's QKV projection + RoPE + append.
void launch_w8a16_gemv_pair(const View& act_x, const View& w0, const View& s0, View& y0,
                            const View& w1, const View& s1, View& y1, int group_size,
                            hipStream_t stream);
void launch_w8a16_gemm_batched(const __half* x, int64_t x_stride, int m, const View& weight,
                               const View& scales, __half* y, int64_t y_stride, int group_size,
                               hipStream_t stream);
void launch_paged_qkv_rope_append(const __half* x, int64_t x_stride, int m, const View& w_qkv,
                                  const View& scales, int group_size, __half* qkv_out,
                                  const af_kv_pool& pool, int layer, const int64_t* d_slots,
                                  const int32_t* d_positions, const float* cos_table,
                                  const float* sin_table, int max_pos, int n_q_heads,
                                  int32_t* d_status, hipStream_t stream);
