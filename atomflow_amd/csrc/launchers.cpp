// launchers.cpp — C++ operator API (include/ops/kernel.h) and ArenaAllocator
// over the C ABI. Errors become std::runtime_error.
#include "ops/kernel.h"

#include <string>

#include "memory/alloc.h"

namespace {

void check(int status, const char* what) {
    if (status != AF_OK)
        throw std::runtime_error(std::string(what) + ": " + af_status_string(status));
}

}  // namespace

void launch_rope(const View& q_input, const View& k_input, const float* cos_cache,
                 const float* sin_cache, int seq_len, int kv_head_num, int q_head_num,
                 int head_dim, hipStream_t stream) {
    // The reference dispatches on the dtype and throws for anything but FP16 /
    // FP8 (rope.cu:62-83); its FP8 branch is never taken by the engine.
    if (q_input.dtype != DataType::FP16 || k_input.dtype != DataType::FP16)
        throw std::runtime_error("Unsupported data type in RoPE");
    check(af_rope(q_input.data_ptr, k_input.data_ptr, cos_cache, sin_cache, seq_len, kv_head_num,
                  q_head_num, head_dim, stream),
          "launch_rope");
}

void launch_cached_attention(const __half* q, const __half* k_cache, const __half* v_cache,
                             __half* out, int seq_len, int head_dim, int n_q_heads,
                             int n_kv_heads, hipStream_t stream) {
    check(af_cached_attention(q, k_cache, v_cache, out, seq_len, head_dim, n_q_heads, n_kv_heads,
                              stream),
          "launch_cached_attention");
}

void launch_write_kv_cache(const View& qkv_out, View& k_cache, View& v_cache, int current_pos,
                           int q_dim, int kv_dim, hipStream_t stream) {
    const int max_seq = int(k_cache.dims[0] < v_cache.dims[0] ? k_cache.dims[0] : v_cache.dims[0]);
    check(af_write_kv_cache(qkv_out.data_ptr, k_cache.data_ptr, v_cache.data_ptr, current_pos,
                            max_seq, q_dim, kv_dim, stream),
          "launch_write_kv_cache");
}

void build_rope_cache(float* d_cos, float* d_sin, int max_seq, int head_dim, float base,
                      hipStream_t stream) {
    check(af_rope_table_build(d_cos, d_sin, max_seq, head_dim, base, stream), "build_rope_cache");
}

void launch_rope_append(View& qkv_out, View& k_cache, View& v_cache, const float* cos_table,
                        const float* sin_table, int pos, const int32_t* d_pos, int n_q_heads,
                        int n_kv_heads, int head_dim, hipStream_t stream) {
    const int max_seq = int(k_cache.dims[0] < v_cache.dims[0] ? k_cache.dims[0] : v_cache.dims[0]);
    check(af_rope_append(qkv_out.data_ptr, k_cache.data_ptr, v_cache.data_ptr, cos_table,
                         sin_table, pos, d_pos, max_seq, n_q_heads, n_kv_heads, head_dim, nullptr,
                         stream),
          "launch_rope_append");
}

void launch_w8a16_gemv(const View& act_x, const View& weight, const View& scales, View& output,
                       int group_size, hipStream_t stream) {
    // Same shape reading as the reference launcher (qkv_gemm.cu:136-139).
    const int n = int(weight.dims[0]);
    const int k = int(weight.dims[1]);
    check(af_w8a16_gemv(act_x.data_ptr, static_cast<const uint8_t*>(weight.data_ptr),
                        scales.data_ptr, output.data_ptr, n, k, group_size, stream),
          "launch_w8a16_gemv");
}

void launch_qkv_rope_append(const View& act_x, const View& w_qkv, const View& scales,
                            int group_size, View& qkv_out, View& k_cache, View& v_cache,
                            const float* cos_table, const float* sin_table, int pos,
                            const int32_t* d_pos, int n_q_heads, int n_kv_heads, int head_dim,
                            hipStream_t stream) {
    const int max_seq = int(k_cache.dims[0] < v_cache.dims[0] ? k_cache.dims[0] : v_cache.dims[0]);
    check(af_qkv_rope_append(act_x.data_ptr, static_cast<const uint8_t*>(w_qkv.data_ptr),
                             scales.data_ptr, int(w_qkv.dims[1]), group_size, qkv_out.data_ptr,
                             k_cache.data_ptr, v_cache.data_ptr, cos_table, sin_table, pos, d_pos,
                             max_seq, n_q_heads, n_kv_heads, head_dim, nullptr, stream),
          "launch_qkv_rope_append");
}

template <typename T>
void launch_tiled_attention_kernel(const T* q_base, const T* k_base, const T* v_base, T* out,
                                   int seq_q, int seq_kv, int head_dim, int n_q_heads,
                                   int n_kv_heads, hipStream_t stream) {
    static_assert(sizeof(T) == 2, "fp16 only, as the reference instantiates it");
    check(af_tiled_attention(q_base, k_base, v_base, out, seq_q, seq_kv, head_dim, n_q_heads,
                             n_kv_heads, stream),
          "launch_tiled_attention_kernel");
}
template void launch_tiled_attention_kernel<__half>(const __half*, const __half*, const __half*,
                                                    __half*, int, int, int, int, int,
                                                    hipStream_t);

void launch_prefill_rope_append(View& qkv_out, int n, View& k_cache, View& v_cache,
                                const float* cos_table, const float* sin_table, int p0,
                                int n_q_heads, int n_kv_heads, int head_dim, hipStream_t stream) {
    const int max_seq = int(k_cache.dims[0] < v_cache.dims[0] ? k_cache.dims[0] : v_cache.dims[0]);
    check(af_prefill_rope_append(qkv_out.data_ptr, n, k_cache.data_ptr, v_cache.data_ptr,
                                 cos_table, sin_table, p0, nullptr, max_seq, n_q_heads, n_kv_heads,
                                 head_dim, nullptr, stream),
          "launch_prefill_rope_append");
}

void launch_prefill_attention(const __half* q, int q_stride, const View& k_cache,
                              const View& v_cache, __half* out, int out_stride, int p0, int n,
                              int kv_len, int n_q_heads, int n_kv_heads, int head_dim,
                              hipStream_t stream) {
    const int max_seq = int(k_cache.dims[0] < v_cache.dims[0] ? k_cache.dims[0] : v_cache.dims[0]);
    check(af_prefill_attention(q, q_stride, k_cache.data_ptr, v_cache.data_ptr, out, out_stride,
                               p0, n, kv_len, max_seq, n_q_heads, n_kv_heads, head_dim, stream),
          "launch_prefill_attention");
}

void launch_paged_prefill_attention(const __half* q, int q_stride, const af_kv_pool& pool,
                                    int layer, const int32_t* d_block_table, int max_blocks,
                                    int p0, int n, int kv_len, __half* out, int out_stride,
                                    int n_q_heads, hipStream_t stream) {
    check(af_paged_prefill_attention(q, q_stride, &pool, layer, d_block_table, max_blocks, p0, n,
                                     kv_len, out, out_stride, n_q_heads, stream),
          "launch_paged_prefill_attention");
}

void launch_prefill_attention_ws(const __half* q, int q_stride, const View& k_cache,
                                 const View& v_cache, __half* out, int out_stride, int p0, int n,
                                 int kv_len, int n_q_heads, int n_kv_heads, int head_dim,
                                 int key_pieces, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
    const int max_seq = int(k_cache.dims[0] < v_cache.dims[0] ? k_cache.dims[0] : v_cache.dims[0]);
    check(af_prefill_attention_ws(q, q_stride, k_cache.data_ptr, v_cache.data_ptr, out, out_stride,
                                  p0, n, kv_len, max_seq, n_q_heads, n_kv_heads, head_dim,
                                  key_pieces, workspace, workspace_bytes, stream),
          "launch_prefill_attention_ws");
}

void launch_paged_prefill_attention_ws(const __half* q, int q_stride, const af_kv_pool& pool,
                                       int layer, const int32_t* d_block_table, int max_blocks,
                                       int p0, int n, int kv_len, __half* out, int out_stride,
                                       int n_q_heads, int key_pieces, void* workspace,
                                       size_t workspace_bytes, hipStream_t stream) {
    check(af_paged_prefill_attention_ws(q, q_stride, &pool, layer, d_block_table, max_blocks, p0,
                                        n, kv_len, out, out_stride, n_q_heads, key_pieces,
                                        workspace, workspace_bytes, stream),
          "launch_paged_prefill_attention_ws");
}

void launch_cached_attention_ws(const __half* q, const __half* k_cache, const __half* v_cache,
                                __half* out, int seq_len, const int32_t* d_seq_len,
                                int max_seq_len, int head_dim, int n_q_heads, int n_kv_heads,
                                int num_splits, void* workspace, size_t workspace_bytes,
                                hipStream_t stream) {
    check(af_cached_attention_ex(q, k_cache, v_cache, out, seq_len, d_seq_len, max_seq_len,
                                 head_dim, n_q_heads, n_kv_heads, num_splits, workspace,
                                 workspace_bytes, stream),
          "launch_cached_attention_ws");
}

void launch_paged_rope_append(__half* qkv_out, int batch, const af_kv_pool& pool, int layer,
                              const int64_t* d_slots, const int32_t* d_positions,
                              const float* cos_table, const float* sin_table, int max_pos,
                              int n_q_heads, hipStream_t stream) {
    check(af_paged_rope_append(qkv_out, batch, &pool, layer, d_slots, d_positions, cos_table,
                               sin_table, max_pos, n_q_heads, stream),
          "launch_paged_rope_append");
}

void launch_paged_attention(const __half* q, int q_stride, const af_kv_pool& pool, int layer,
                            const int32_t* d_block_tables, int max_blocks_per_seq,
                            const int32_t* d_seq_lens, int batch, int max_seq_len, __half* out,
                            int out_stride, int n_q_heads, int num_splits, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
    check(af_paged_attention(q, q_stride, &pool, layer, d_block_tables, max_blocks_per_seq,
                             d_seq_lens, batch, max_seq_len, out, out_stride, n_q_heads,
                             num_splits, workspace, workspace_bytes, stream),
          "launch_paged_attention");
}

void launch_kv_copy_blocks(const af_kv_pool& pool, const int32_t* d_copies, const int32_t* d_count,
                           int max_copies, hipStream_t stream) {
    check(af_kv_copy_blocks(&pool, d_copies, d_count, max_copies, stream), "launch_kv_copy_blocks");
}

void launch_paged_decode_fused(__half* qkv_out, int batch, const af_kv_pool& pool, int layer,
                               const int64_t* d_slots, const int32_t* d_positions,
                               const float* cos_table, const float* sin_table, int max_pos,
                               const int32_t* d_block_tables, int max_blocks_per_seq,
                               int max_seq_len, __half* out, int out_stride, int n_q_heads,
                               int num_splits, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
    check(af_paged_decode_fused(qkv_out, batch, &pool, layer, d_slots, d_positions, cos_table,
                                sin_table, max_pos, d_block_tables, max_blocks_per_seq,
                                max_seq_len, out, out_stride, n_q_heads, num_splits, workspace,
                                workspace_bytes, stream),
          "launch_paged_decode_fused");
}

void launch_paged_attention_shared_prefix(const __half* q, int q_stride, const af_kv_pool& pool,
                                          int layer, const int32_t* d_prefix_table,
                                          int prefix_len, int prefix_splits,
                                          const int32_t* d_block_tables, int max_blocks_per_seq,
                                          const int32_t* d_seq_lens, int batch, int max_seq_len,
                                          __half* out, int out_stride, int n_q_heads,
                                          int num_splits, void* workspace, size_t workspace_bytes,
                                          hipStream_t stream) {
    check(af_paged_attention_shared_prefix(q, q_stride, &pool, layer, d_prefix_table, prefix_len,
                                           prefix_splits, d_block_tables, max_blocks_per_seq,
                                           d_seq_lens, batch, max_seq_len, out, out_stride,
                                           n_q_heads, num_splits, workspace, workspace_bytes,
                                           stream),
          "launch_paged_attention_shared_prefix");
}

void launch_paged_decode_fused_shared_prefix(
    __half* qkv_out, int batch, const af_kv_pool& pool, int layer, const int64_t* d_slots,
    const int32_t* d_positions, const float* cos_table, const float* sin_table, int max_pos,
    const int32_t* d_prefix_table, int prefix_len, int prefix_splits,
    const int32_t* d_block_tables, int max_blocks_per_seq, int max_seq_len, __half* out,
    int out_stride, int n_q_heads, int num_splits, void* workspace, size_t workspace_bytes,
    hipStream_t stream) {
    check(af_paged_decode_fused_shared_prefix(
              qkv_out, batch, &pool, layer, d_slots, d_positions, cos_table, sin_table, max_pos,
              d_prefix_table, prefix_len, prefix_splits, d_block_tables, max_blocks_per_seq,
              max_seq_len, out, out_stride, n_q_heads, num_splits, workspace, workspace_bytes,
              stream),
          "launch_paged_decode_fused_shared_prefix");
}

void launch_w8a16_gemv_pair(const View& act_x, const View& w0, const View& s0, View& y0,
                            const View& w1, const View& s1, View& y1, int group_size,
                            hipStream_t stream) {
    check(af_w8a16_gemv_pair(act_x.data_ptr, static_cast<const uint8_t*>(w0.data_ptr),
                             s0.data_ptr, y0.data_ptr, int(w0.dims[0]),
                             static_cast<const uint8_t*>(w1.data_ptr), s1.data_ptr, y1.data_ptr,
                             int(w1.dims[0]), int(w0.dims[1]), group_size, stream),
          "launch_w8a16_gemv_pair");
}

void launch_w8a16_gemm_batched(const __half* x, int64_t x_stride, int m, const View& weight,
                               const View& scales, __half* y, int64_t y_stride, int group_size,
                               hipStream_t stream) {
    check(af_w8a16_gemm_batched(x, x_stride, m, static_cast<const uint8_t*>(weight.data_ptr),
                                scales.data_ptr, y, y_stride, int(weight.dims[0]),
                                int(weight.dims[1]), group_size, stream),
          "launch_w8a16_gemm_batched");
}

void launch_paged_qkv_rope_append(const __half* x, int64_t x_stride, int m, const View& w_qkv,
                                  const View& scales, int group_size, __half* qkv_out,
                                  const af_kv_pool& pool, int layer, const int64_t* d_slots,
                                  const int32_t* d_positions, const float* cos_table,
                                  const float* sin_table, int max_pos, int n_q_heads,
                                  int32_t* d_status, hipStream_t stream) {
    check(af_paged_qkv_rope_append(x, x_stride, m, static_cast<const uint8_t*>(w_qkv.data_ptr),
                                   scales.data_ptr, int(w_qkv.dims[1]), group_size, qkv_out,
                                   &pool, layer, d_slots, d_positions, cos_table, sin_table,
                                   max_pos, n_q_heads, d_status, stream),
          "launch_paged_qkv_rope_append");
}

ArenaAllocator::ArenaAllocator(size_t total_size) {
    capacity_ = align_to_128(total_size);
    offset_ = 0;
    if (hipMalloc(&base_ptr_, capacity_) != hipSuccess) {
        base_ptr_ = nullptr;
        throw std::runtime_error("ArenaAllocator: failed to allocate " +
                                 std::to_string(capacity_ >> 20) + " MB");
    }
    owns_ = true;
}

ArenaAllocator::~ArenaAllocator() {
    if (owns_ && base_ptr_) (void)hipFree(base_ptr_);
}
