/*
 * af_kv.h — C ABI of the MI355X KV-cache hot path (libatomflow_kv.so).
 *
 * Plain C: raw device pointers, integer sizes, a stream handle. No C++ or torch
 * types. Every function returns an int status:
 *     0            success (AF_OK)
 *     > 0          a hipError_t value from the HIP runtime
 *     < 0          an AF_ERR_* code below
 * The ABI never throws and never aborts. Kernel launches are asynchronous and
 * stream-ordered, do no host synchronisation and allocate nothing, so they may
 * be recorded into a hipGraph (stream capture). Device buffers are owned by the
 * caller unless a function says otherwise.
 *
 * Conventions shared with the reference (Altersieg/AtomFlow):
 *   qkv_out row    = [Q: n_q_heads*head_dim | K: kv_dim | V: kv_dim] fp16
 *                    (src/core/engine.cu:326-331, include/core/model_state.h:48)
 *   KV cache row t = [kv_head 0 dims 0..hd-1 | kv_head 1 ... ], kv_dim = n_kv_heads*head_dim
 *                    (include/core/model_state.h:56-64, README.md:57)
 *   GQA mapping    = kv_head(h) = h * n_kv_heads / n_q_heads (src/kernel/tiled_attention.cu:208)
 *   RoPE pairs     = (d, d + head_dim/2), table row `pos` = pos * head_dim/2 floats
 *                    (src/kernel/rope.cu:22-45, src/kernel/helpers.cu:94-113)
 */
#ifndef AF_KV_H_
#define AF_KV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
#define AF_OK 0
/* -1 is the value the reference's BlockManager::allocate_block() returns when
 * the pool is exhausted (src/experimental/server_arch/paged_kv_manager.h:105-107). */
#define AF_ERR_POOL_EXHAUSTED (-1)
#define AF_ERR_INVALID_ARG (-2)     /* null pointer, bad size, inconsistent shapes   */
#define AF_ERR_UNSUPPORTED (-3)     /* head_dim / GQA ratio / dtype not compiled in  */
#define AF_ERR_OUT_OF_RANGE (-4)    /* position >= capacity, table too short          */
#define AF_ERR_BAD_BLOCK (-5)       /* block id out of range or already free          */
#define AF_ERR_WORKSPACE (-6)       /* workspace missing or too small                 */
#define AF_ERR_BAD_SEQUENCE (-7)    /* unknown sequence id                            */
#define AF_ERR_NOT_BUILT (-8)       /* library built without a device code object     */
#define AF_ERR_BAD_FILE (-9)        /* weight file missing, not AtomFlow, or truncated */
#define AF_ERR_TIMEOUT (-10)        /* a decode-attention split never published (output NaN) */

typedef void* af_stream_t; /* hipStream_t; NULL = the default stream */

/* KV element types; values equal the reference's DataType enumerators
 * (include/core/view.h:15-20). */
#define AF_KV_FP16 1
#define AF_KV_FP8_E4M3 3

const char* af_status_string(int status);
/* (major << 16) | (minor << 8) | patch */
int af_version(void);

/* ======================================================================== */
/* a1. RoPE cos/sin table                                                    */
/* ======================================================================== */
/* Replaces build_rope_cache (include/ops/kernel.h:195-197, src/kernel/helpers.cu:94-113).
 * Table layout [max_seq, head_dim/2] fp32; computed on the host in float
 * (theta = s / powf(base, 2*i/head_dim); cosf/sinf) and copied to the device.
 * The copy is synchronous with respect to the host (the host staging buffer is
 * released on return). */
int af_rope_table_build(float* d_cos, float* d_sin, int max_seq, int head_dim, float base,
                        af_stream_t stream);
/* Same table into host memory (no device needed). */
int af_rope_table_host(float* h_cos, float* h_sin, int max_seq, int head_dim, float base);

/* ======================================================================== */
/* a2 / a3. Reference-shaped RoPE and KV write                              */
/* ======================================================================== */
/* Replaces launch_rope (include/ops/kernel.h:32-42, src/kernel/rope.cu:48-84).
 * q: [seq_len, q_head_num*head_dim] fp16, k: [seq_len, kv_head_num*head_dim]
 * fp16, both rotated in place; cos/sin: table rows starting at the position of
 * token 0 (the engine passes d_cos + pos*head_dim/2, src/core/engine.cu:340-344). */
int af_rope(void* q, void* k, const float* cos_cache, const float* sin_cache, int seq_len,
            int kv_head_num, int q_head_num, int head_dim, af_stream_t stream);

/* Replaces launch_write_kv_cache (include/ops/kernel.h:167-174, src/kernel/helpers.cu:141-156).
 * k_cache[current_pos, :] = qkv_out[q_dim : q_dim+kv_dim],
 * v_cache[current_pos, :] = qkv_out[q_dim+kv_dim : q_dim+2*kv_dim].
 * max_seq (the cache's row count) is checked: current_pos >= max_seq -> AF_ERR_OUT_OF_RANGE. */
int af_write_kv_cache(const void* qkv_out, void* k_cache, void* v_cache, int current_pos,
                      int max_seq, int q_dim, int kv_dim, af_stream_t stream);

/* ======================================================================== */
/* a2+a3 fused. RoPE + append into the contiguous cache (one launch)         */
/* ======================================================================== */
/* Equivalent to launch_rope(pos) followed by launch_write_kv_cache(pos)
 * (src/core/engine.cu:326-355): Q and K inside qkv_out are rotated in place,
 * then K (rotated) and V are written to row pos of k_cache / v_cache.
 * Position: *d_pos when d_pos != NULL (device-resident, for graph replay),
 * otherwise `pos`. A device-resident pos >= max_seq writes nothing and stores
 * AF_ERR_OUT_OF_RANGE into *d_status when d_status != NULL. */
int af_rope_append(void* qkv_out, void* k_cache, void* v_cache, const float* cos_table,
                   const float* sin_table, int pos, const int32_t* d_pos, int max_seq,
                   int n_q_heads, int n_kv_heads, int head_dim, int32_t* d_status,
                   af_stream_t stream);

/* ======================================================================== */
/* a5. GQA decode attention over the contiguous cache                       */
/* ======================================================================== */
/* Replaces launch_cached_attention (include/ops/kernel.h:93-103,
 * src/kernel/tiled_attention.cu:275-296), same arguments. Split-K over the
 * sequence with a library-owned workspace (allocated on the first call per
 * device; call af_attention_reserve() first when the call will be captured).
 * Combiner timeout: with the default split count (2..32 splits for up to 16 KV
 * heads, head_dim 128, up to 4 query heads per KV head) one combiner workgroup
 * per KV head merges the splits' partials, waiting on each split's ready flag
 * with a bounded poll (about a second). Forward progress rests on in-order
 * workgroup dispatch: the combiners have the highest workgroup ids, so every
 * split is resident before a combiner waits. If a split never publishes, the
 * affected outputs are NaN; this entry point has no status argument, so NaN
 * is the only signal (af_decode_attention_fused also stores AF_ERR_TIMEOUT).
 * A combiner that gives up poisons the workspace: every later launch on it
 * returns NaN for the pairs the combiner merges (and AF_ERR_TIMEOUT where there
 * is a status) until af_attention_workspace_init clears it, because a split of
 * the failed launch may still set a flag that a later launch would trust. The
 * library-owned workspace of this entry point (and the static array of the
 * _noalloc form) then stays poisoned until the process ends: a timeout means
 * the device left a resident workgroup unrun for about a second. */
int af_cached_attention(const void* q, const void* k_cache, const void* v_cache, void* out,
                        int seq_len, int head_dim, int n_q_heads, int n_kv_heads,
                        af_stream_t stream);

/* Allocation-free form of af_cached_attention (same arguments, same split
 * count, same results). No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under hipGraph stream capture, serving
 * loops and harnesses that forbid hipMalloc). The split-K workspace is a static
 * device array of af_cached_attention_noalloc_max_bytes() bytes per device
 * (4.125 MiB), held until the process ends; its address is looked up with
 * hipGetSymbolAddress on the first call on a device, which also clears its
 * arrival counters with a fill kernel on `stream`. No hipMalloc / hipFree.
 * Shapes whose workspace exceeds the array (attn workspace of batch 1,
 * n_q_heads, head_dim, default splits for seq_len) return AF_ERR_WORKSPACE.
 * Every call on one device shares that array: calls that may overlap on one
 * device (different streams, no ordering) race and must not be issued. */
int af_cached_attention_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                void* out, int seq_len, int head_dim, int n_q_heads,
                                int n_kv_heads, af_stream_t stream);
size_t af_cached_attention_noalloc_max_bytes(void);

/* Pre-allocates the library-owned workspace for batch x n_q_heads heads. */
int af_attention_reserve(int batch, int n_q_heads, int n_kv_heads, int head_dim);

/* Workspace bytes for the explicit-workspace entry points. */
size_t af_attention_workspace_size(int batch, int n_q_heads, int n_kv_heads, int head_dim,
                                   int num_splits);
/* Zero-fills a workspace (a fill kernel, not a memset node). Needed once after
 * allocation; every attention launch leaves its counters at zero again, except
 * after a combiner timeout, which leaves the workspace poisoned (see
 * af_cached_attention) until this is called again. */
int af_attention_workspace_init(void* workspace, size_t workspace_bytes, af_stream_t stream);
/* Split count the library picks for a given longest sequence and batch. */
int af_attention_default_splits(int max_seq_len, int batch, int n_kv_heads);

/* Explicit-workspace form. seq_len: used when d_seq_len == NULL; otherwise the
 * length is read on the device (graph replay). num_splits <= 0 picks the
 * default for max_seq_len. k/v row stride is n_kv_heads*head_dim. With 2..32
 * splits, n_kv_heads <= 16, head_dim 128 and up to 4 query heads per KV head,
 * one combiner workgroup per KV head merges the splits' partials as they are
 * published (a combiner that waits about a second for a split that never
 * publishes writes NaN; the fused form then stores AF_ERR_TIMEOUT; see
 * af_cached_attention for the dispatch-order rule it rests on). */
int af_cached_attention_ex(const void* q, const void* k_cache, const void* v_cache, void* out,
                           int seq_len, const int32_t* d_seq_len, int max_seq_len, int head_dim,
                           int n_q_heads, int n_kv_heads, int num_splits, void* workspace,
                           size_t workspace_bytes, af_stream_t stream);

/* One-launch decode layer step: af_rope_append(pos) followed by
 * af_cached_attention_ex(seq_len = pos + 1) fused into one kernel
 * (src/core/engine.cu:326-370 issues them as three launches). Same outputs bit
 * for bit as the two separate calls with the same num_splits: Q and K rotated
 * in place in qkv_out, rotated K and V written to row pos, attention into out.
 * Position: *d_pos when d_pos != NULL, else pos; a device position >= max_seq
 * writes nothing and stores AF_ERR_OUT_OF_RANGE into *d_status (if given). */
int af_decode_attention_fused(void* qkv_out, void* k_cache, void* v_cache, const float* cos_table,
                              const float* sin_table, int pos, const int32_t* d_pos, int max_seq,
                              void* out, int n_q_heads, int n_kv_heads, int head_dim,
                              int num_splits, void* workspace, size_t workspace_bytes,
                              int32_t* d_status, af_stream_t stream);

/* ======================================================================== */
/* a6-a8. Paged KV pool                                                      */
/* ======================================================================== */
/* One device allocation holds every layer (one block id spans all layers):
 *   base = [layer 0 K | layer 0 V | layer 1 K | ... ], each slab
 *          total_blocks * block_size * kv_dim elements,
 *   block b of layer l, K row r at
 *          base + ((2*l) * total_blocks + b) * block_size * kv_dim + r * kv_dim.
 * FP8 pools carry fp32 scales [n_layers][2 (K,V)][n_kv_heads]; element value =
 * e4m3fn(code) * scale (convention of tools/quantize_weights.py:249-260). */
typedef struct af_kv_pool {
    void* base;
    const float* scales; /* FP8 only, else NULL */
    int32_t dtype;       /* AF_KV_FP16 or AF_KV_FP8_E4M3 */
    int32_t block_size;  /* tokens per block, power of two, >= 8 */
    int32_t n_layers;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t flags;       /* AF_KV_POOL_* bits; 0 for none */
    int64_t total_blocks;
} af_kv_pool;

/* af_kv_pool.flags: the block tables of one launch may map the same block for
 * several sequences (forked sequences, prefix caching). Decode attention then
 * reads KV rows with the ordinary cache policy, so the sequences after the first
 * find shared rows in L2; without it, rows are read with non-temporal loads
 * (each row once per launch), which streams faster. Either way the results are
 * the same bits. Other bits are rejected (AF_ERR_INVALID_ARG). */
#define AF_KV_POOL_SHARED_BLOCKS 1

size_t af_kv_pool_bytes(const af_kv_pool* pool);

/* Paged RoPE + append for a batch (the paged form of af_rope_append).
 * qkv_out: [batch, q_dim + 2*kv_dim] fp16 (rows contiguous).
 * d_positions[b]: the logical position of the new token (RoPE row).
 * d_slots[b]: physical row = block_id * block_size + offset (from the BlockManager).
 * FP8 pools quantise K/V with the layer's scales (RNE, clamped to +-448). */
int af_paged_rope_append(void* qkv_out, int batch, const af_kv_pool* pool, int layer,
                         const int64_t* d_slots, const int32_t* d_positions,
                         const float* cos_table, const float* sin_table, int max_pos,
                         int n_q_heads, af_stream_t stream);

/* Paged GQA decode attention for a batch.
 * q: [batch, q_stride] fp16 (head h at q + b*q_stride + h*head_dim),
 * d_block_tables: [batch, max_blocks_per_seq] int32, d_seq_lens: [batch] int32,
 * out: [batch, out_stride] fp16. max_seq_len bounds every d_seq_lens[b] and sizes
 * the split grid. Workspace from af_attention_workspace_size(batch, ...).
 * With num_splits = 0, batches of FP8 pools (batch * n_kv_heads * 2 >= CUs,
 * batch <= 256, head_dim 128) run as one persistent launch whose workgroups
 * claim row ranges from a counter in the workspace (re-armed by the launch). */
int af_paged_attention(const void* q, int q_stride, const af_kv_pool* pool, int layer,
                       const int32_t* d_block_tables, int max_blocks_per_seq,
                       const int32_t* d_seq_lens, int batch, int max_seq_len, void* out,
                       int out_stride, int n_q_heads, int num_splits, void* workspace,
                       size_t workspace_bytes, af_stream_t stream);

/* Paged decode layer step in one launch: af_paged_rope_append followed by
 * af_paged_attention with d_seq_lens[b] = d_positions[b] + 1 (the block tables
 * already map the new position to d_slots[b], as af_bm_plan_decode leaves
 * them). qkv_out rows are [batch, (n_q_heads + 2 n_kv_heads) * head_dim]. */
int af_paged_decode_fused(void* qkv_out, int batch, const af_kv_pool* pool, int layer,
                          const int64_t* d_slots, const int32_t* d_positions,
                          const float* cos_table, const float* sin_table, int max_pos,
                          const int32_t* d_block_tables, int max_blocks_per_seq, int max_seq_len,
                          void* out, int out_stride, int n_q_heads, int num_splits,
                          void* workspace, size_t workspace_bytes, af_stream_t stream);

/* Shared-prefix ("cascade") form of af_paged_attention for a batch whose
 * sequences all begin with the same prefix_len rows (forks of one prompt under
 * copy-on-write, src/experimental/server_arch/paged_kv_manager.h:51,61: the
 * reference reads the shared blocks once per sequence through its tables). Same
 * result as af_paged_attention, within its tolerance, when rows
 * [0, prefix_len) of every sequence hold the values d_prefix_table maps
 * (one row of max_blocks_per_seq entries, e.g. the root sequence's table).
 * The prefix is attended once for the whole batch on the matrix cores (one
 * launch, prefix_splits key ranges; 0 = default), the per-sequence rows
 * [prefix_len, L) by the split-K decode kernel, whose combine merges both.
 * head_dim 128. A sequence with L == prefix_len attends the prefix records
 * alone; one with L < prefix_len attends its own rows [0, L) through its table
 * and leaves the prefix records out, so every L gets af_paged_attention's
 * result (rows [0, L) of its table must then hold the prefix's first L rows).
 * Workspace: af_attention_workspace_size(batch, ..., num_splits +
 * prefix_splits); one sized with num_splits = 0 (the maximum) always fits.
 * No counterpart entry in the reference (an optimisation of the same op). */
int af_paged_attention_shared_prefix(const void* q, int q_stride, const af_kv_pool* pool,
                                     int layer, const int32_t* d_prefix_table, int prefix_len,
                                     int prefix_splits, const int32_t* d_block_tables,
                                     int max_blocks_per_seq, const int32_t* d_seq_lens, int batch,
                                     int max_seq_len, void* out, int out_stride, int n_q_heads,
                                     int num_splits, void* workspace, size_t workspace_bytes,
                                     af_stream_t stream);

/* af_paged_decode_fused with a shared prefix: the prefix launch rotates its own
 * copy of each query (same arithmetic), then the fused decode launch ropes,
 * appends and attends rows [prefix_len, pos] and merges the prefix partials.
 * Outputs as af_paged_decode_fused (qkv_out, pool rows bit for bit; attention
 * within tolerance). */
int af_paged_decode_fused_shared_prefix(void* qkv_out, int batch, const af_kv_pool* pool,
                                        int layer, const int64_t* d_slots,
                                        const int32_t* d_positions, const float* cos_table,
                                        const float* sin_table, int max_pos,
                                        const int32_t* d_prefix_table, int prefix_len,
                                        int prefix_splits, const int32_t* d_block_tables,
                                        int max_blocks_per_seq, int max_seq_len, void* out,
                                        int out_stride, int n_q_heads, int num_splits,
                                        void* workspace, size_t workspace_bytes,
                                        af_stream_t stream);

/* Gathers one sequence's first seq_len logical rows of `layer` into
 * contiguous [seq_len, kv_dim] buffers (K and V; elements copied bit for bit). */
int af_paged_gather(const af_kv_pool* pool, int layer, const int32_t* d_block_table,
                    int seq_len, void* k_dst, void* v_dst, af_stream_t stream);

/* Copy-on-write block copies for every layer: for i < *d_count (device int),
 * rows [0, d_copies[3i+2]) of block d_copies[3i] are copied to block
 * d_copies[3i+1], K and V, all layers. max_copies bounds *d_count. */
int af_kv_copy_blocks(const af_kv_pool* pool, const int32_t* d_copies, const int32_t* d_count,
                      int max_copies, af_stream_t stream);

/* FP8 E4M3 quantisation of fp16 values with one fp32 scale (device). */
int af_fp8_quantize(const void* src_f16, uint8_t* dst, size_t n, float scale, af_stream_t stream);

/* ======================================================================== */
/* b1. W8A16 GEMV either side of the path (QKV projection, output proj.)   */
/* ======================================================================== */
/* Replaces launch_w8a16_gemv (include/ops/kernel.h:138-145,
 * src/kernel/qkv_gemm.cu:32-152): y[n] = sum_k e4m3(weight[n,k]) *
 * scales[n, k/group_size] * x[k], fp32 accumulation, fp16 output.
 * x: [k] fp16, weight: [n, k] E4M3 codes row-major, scales: [n, k/group_size]
 * fp16, y: [n] fp16. k and group_size multiples of 16 (the engine uses 128);
 * x and weight 16-byte aligned. */
int af_w8a16_gemv(const void* x, const uint8_t* weight, const void* scales, void* y, int n, int k,
                  int group_size, af_stream_t stream);
/* Two af_w8a16_gemv of the same activation in one launch: y0 = W0 x (n0 rows)
 * and y1 = W1 x (n1 rows), each bit for bit the single call's output. For the
 * MLP's gate and up projections, which the engine issues as two launches of
 * launch_w8a16_gemv on the same input (src/core/engine.cu:418-436). */
int af_w8a16_gemv_pair(const void* x, const uint8_t* weight0, const void* scales0, void* y0, int n0,
                       const uint8_t* weight1, const void* scales1, void* y1, int n1, int k,
                       int group_size, af_stream_t stream);

/* The W8A16 projection of m tokens (rows of x, x_stride elements apart) in one
 * launch: y[i] = af_w8a16_gemv(x[i]) for every token i, within the same fp32
 * summation bound (no counterpart in the reference, whose engine decodes one
 * token per step: launch_w8a16_gemv, qkv_gemm.cu:32-152; a serving step has one
 * token per sequence). k and group_size multiples of 32; x_stride >= k and a
 * multiple of 8; x and weight 16-byte aligned. Weights are read once per 32
 * tokens; m = 1 runs af_w8a16_gemv itself (the same bits). */
int af_w8a16_gemm_batched(const void* x, int64_t x_stride, int m, const uint8_t* weight,
                          const void* scales, void* y, int64_t y_stride, int n, int k,
                          int group_size, af_stream_t stream);

/* The paged serving step's QKV projection + RoPE + KV append in one launch:
 * af_w8a16_gemm_batched of the fused QKV weight into qkv_out ([m][q_dim +
 * 2 kv_dim]) followed by af_paged_rope_append(qkv_out, m, pool, layer, d_slots,
 * d_positions, ...), the same outputs bit for bit (the paged form of
 * af_qkv_rope_append). A token whose position or slot is out of range gets its
 * unrotated projection in qkv_out, nothing in the pool, and AF_ERR_OUT_OF_RANGE
 * in *d_status (if given). head_dim 128. m = 1 runs the single-token form of
 * af_qkv_rope_append on the pool row (the GEMV's arithmetic, which is what
 * af_w8a16_gemm_batched computes at m = 1). */
int af_paged_qkv_rope_append(const void* x, int64_t x_stride, int m, const uint8_t* w_qkv,
                             const void* scales, int k, int group_size, void* qkv_out,
                             const af_kv_pool* pool, int layer, const int64_t* d_slots,
                             const int32_t* d_positions, const float* cos_table,
                             const float* sin_table, int max_pos, int n_q_heads,
                             int32_t* d_status, af_stream_t stream);

/* Decode QKV projection, RoPE and KV append in one launch: af_w8a16_gemv of the
 * fused QKV weight into qkv_out ([Q | K | V] heads, the engine's layout,
 * src/core/engine.cu:310-331) followed by af_rope_append(pos) — the same
 * outputs bit for bit (src/core/engine.cu:315-355 issues the three launches).
 * Position: *d_pos when d_pos != NULL, else pos; a device position >= max_seq
 * writes nothing and stores AF_ERR_OUT_OF_RANGE into *d_status (if given).
 * head_dim even. */
int af_qkv_rope_append(const void* x, const uint8_t* w_qkv, const void* scales, int k,
                       int group_size, void* qkv_out, void* k_cache, void* v_cache,
                       const float* cos_table, const float* sin_table, int pos,
                       const int32_t* d_pos, int max_seq, int n_q_heads, int n_kv_heads,
                       int head_dim, int32_t* d_status, af_stream_t stream);

/* ======================================================================== */
/* b2. Prefill: multi-token append and causal attention over a prompt chunk */
/* ======================================================================== */
/* Multi-token form of af_rope_append: n rows of qkv_out ([n, (n_q_heads +
 * 2*n_kv_heads)*head_dim], the QKV projection of n prompt tokens) get RoPE with
 * table rows p0 .. p0+n-1 (rope.cu:22-45 with seq_len = n, rope.cu:59-60) and
 * their K/V rows are written to cache rows p0 .. p0+n-1 (helpers.cu:126-139 per
 * token). Start position: *d_p0 when d_p0 != NULL, else p0. With a host p0 the
 * whole chunk must fit (p0 + n <= max_seq, else AF_ERR_OUT_OF_RANGE and nothing
 * is launched); with a device p0 each row past max_seq is skipped and
 * AF_ERR_OUT_OF_RANGE is stored into *d_status (if given). */
int af_prefill_rope_append(void* qkv_out, int n, void* k_cache, void* v_cache,
                           const float* cos_table, const float* sin_table, int p0,
                           const int32_t* d_p0, int max_seq, int n_q_heads, int n_kv_heads,
                           int head_dim, int32_t* d_status, af_stream_t stream);

/* Causal GQA attention of a chunk of n query tokens at cache positions
 * p0 .. p0+n-1 over the contiguous cache: query i attends cache rows
 * [0, min(p0 + i + 1, kv_len)). Generalises gqa_attention_kernel
 * (src/kernel/tiled_attention.cu:34-130), whose form is p0 = 0, kv_len = seq_kv.
 * q: row i at q + i*q_stride (elements), head h at +h*head_dim (the roped Q of
 * af_prefill_rope_append's qkv_out has q_stride = (n_q_heads+2*n_kv_heads)*head_dim);
 * k_cache/v_cache: [max_seq, n_kv_heads*head_dim]; out: row i at
 * out + i*out_stride. head_dim 128 (else AF_ERR_UNSUPPORTED); 1 <= kv_len <= max_seq.
 * fp16 in and out; scores and softmax in fp32, probabilities rounded to fp16 for
 * the P.V product, fp32 accumulation. */
int af_prefill_attention(const void* q, int q_stride, const void* k_cache, const void* v_cache,
                         void* out, int out_stride, int p0, int n, int kv_len, int max_seq,
                         int n_q_heads, int n_kv_heads, int head_dim, af_stream_t stream);

/* af_prefill_attention over one sequence's rows of a paged pool: logical row t of
 * `layer` is read through d_block_table (device int32 [max_blocks]), slot
 * d_block_table[t / block_size] * block_size + t % block_size. Chunked prefill
 * (src/experimental/server_arch roadmap, README.md:269): append the chunk with
 * af_paged_rope_append (one slot per token), then this. FP16 or FP8-E4M3 pools
 * (FP8: codes convert to fp16 exactly, the layer's K scale multiplies the scores
 * and its V scale the output), head_dim 128 (else AF_ERR_UNSUPPORTED);
 * kv_len <= max_blocks * block_size. */
int af_paged_prefill_attention(const void* q, int q_stride, const af_kv_pool* pool, int layer,
                               const int32_t* d_block_table, int max_blocks, int p0, int n,
                               int kv_len, void* out, int out_stride, int n_q_heads,
                               af_stream_t stream);

/* af_prefill_attention / af_paged_prefill_attention with key pieces (same
 * arguments, results and rules; no counterpart in the reference). A chunk's
 * query tiles (128 queries) attend unequal key ranges under the causal mask;
 * a tile with more key tiles (64 keys) than one workgroup slot's share of the
 * chunk's work is cut into up to four key ranges, each a workgroup, and the
 * last of them to finish merges the pieces (online-softmax merge in piece
 * order, so the output does not depend on which finishes last). key_pieces:
 * 0 = the library's choice, 1 = no cut (bit-identical to the entry points
 * above), 2..4 = at most that many pieces per tile. workspace: at least
 * af_prefill_workspace_size(p0, n, kv_len, n_q_heads, key_pieces) bytes,
 * 256-B aligned, zero-filled once by af_attention_workspace_init (each launch
 * leaves its counters at zero); launches sharing a workspace must be ordered
 * (one stream). AF_ERR_WORKSPACE if it is missing or too small when a cut is
 * planned. */
int af_prefill_attention_ws(const void* q, int q_stride, const void* k_cache, const void* v_cache,
                            void* out, int out_stride, int p0, int n, int kv_len, int max_seq,
                            int n_q_heads, int n_kv_heads, int head_dim, int key_pieces,
                            void* workspace, size_t workspace_bytes, af_stream_t stream);
int af_paged_prefill_attention_ws(const void* q, int q_stride, const af_kv_pool* pool, int layer,
                                  const int32_t* d_block_table, int max_blocks, int p0, int n,
                                  int kv_len, void* out, int out_stride, int n_q_heads,
                                  int key_pieces, void* workspace, size_t workspace_bytes,
                                  af_stream_t stream);
/* Workspace bytes of the _ws prefill entry points for one chunk (0 on bad
 * arguments). */
size_t af_prefill_workspace_size(int p0, int n, int kv_len, int n_q_heads, int key_pieces);

/* Several chunks (of different sequences) in one launch, the per-layer form of a
 * serving step's chunked prefill. d_chunks: device int32 [n_chunks][4] =
 * (p0, n, kv_len, row0): chunk c's queries are rows row0 .. row0+n-1 of q and out;
 * d_tables: device int32 [n_chunks][max_blocks], chunk c's block table;
 * d_tile_map: device int32 [n_tiles][2] from af_prefill_tile_map. Per-chunk
 * semantics as af_paged_prefill_attention; outputs equal one launch per chunk
 * bit for bit. The descriptors are device data and are not validated. */
int af_paged_prefill_attention_batched(const void* q, int q_stride, const af_kv_pool* pool,
                                       int layer, const int32_t* d_tables, int max_blocks,
                                       const int32_t* d_chunks, const int32_t* d_tile_map,
                                       int n_tiles, void* out, int out_stride, int n_q_heads,
                                       af_stream_t stream);
/* Host helper: the query tiles (128 queries each) of the chunks h_chunks (same
 * layout as d_chunks), heaviest first, into h_tile_map [max_tiles][2] = (chunk,
 * tile). Returns the tile count, or AF_ERR_WORKSPACE when it exceeds max_tiles. */
int af_prefill_tile_map(const int32_t* h_chunks, int n_chunks, int32_t* h_tile_map,
                        int max_tiles);
/* Key pieces for the batched launch (no counterpart in the reference): as
 * af_prefill_tile_map, but when the launch's tiles x n_q_heads are fewer than
 * the device's workgroup slots (two per CU), heavy tiles are cut into up to
 * key_pieces (0 = 4) key ranges, with the rule of af_prefill_attention_ws.
 * h_map [max_entries][4] = (chunk, tile, piece | pieces << 8, tile index),
 * heaviest piece first. Returns the entry count (AF_ERR_WORKSPACE when it
 * exceeds max_entries) and sets *n_groups (tiles), *max_pieces and the
 * workspace bytes af_paged_prefill_attention_batched_ws needs. */
int af_prefill_piece_map(const int32_t* h_chunks, int n_chunks, int n_q_heads, int key_pieces,
                         int32_t* h_map, int max_entries, int* n_groups, int* max_pieces,
                         size_t* workspace_bytes);
/* af_paged_prefill_attention_batched over a piece map (d_piece_map: the
 * uploaded h_map, n_entries, n_groups and max_pieces as af_prefill_piece_map
 * returned them). Cut tiles merge their pieces as af_prefill_attention_ws does;
 * the workspace rules are the same (zeroed once, ordered launches). */
int af_paged_prefill_attention_batched_ws(const void* q, int q_stride, const af_kv_pool* pool,
                                          int layer, const int32_t* d_tables, int max_blocks,
                                          const int32_t* d_chunks, const int32_t* d_piece_map,
                                          int n_entries, int n_groups, int max_pieces, void* out,
                                          int out_stride, int n_q_heads, void* workspace,
                                          size_t workspace_bytes, af_stream_t stream);

/* launch_tiled_attention_kernel<half> (include/ops/kernel.h:73-85,
 * src/kernel/tiled_attention.cu:136-161): q [seq_q, n_q_heads*head_dim],
 * k/v [seq_kv, n_kv_heads*head_dim], out [seq_q, n_q_heads*head_dim]; query i
 * attends keys s <= i, s < seq_kv. seq_kv = 0 writes zeros, as the reference's
 * empty accumulation does. */
int af_tiled_attention(const void* q, const void* k, const void* v, void* out, int seq_q,
                       int seq_kv, int head_dim, int n_q_heads, int n_kv_heads,
                       af_stream_t stream);

/* ======================================================================== */
/* a6. BlockManager (host bookkeeping, optional device pool)                */
/* ======================================================================== */
/* Contract of atomflow::server::BlockManager
 * (src/experimental/server_arch/paged_kv_manager.h:90-121), extended with
 * refcounts, sequences (PageTables), fork and copy-on-write. Not thread-safe. */
typedef struct af_block_manager af_block_manager;

/* allocate_pool = 1: one hipMalloc for the pool, like BlockManager::initialize
 * (paged_kv_manager.h:103); 0: host bookkeeping only (the pool may be given
 * later with af_bm_attach_pool). */
int af_bm_create(int total_blocks, int block_size, int n_layers, int n_kv_heads, int head_dim,
                 int dtype, int allocate_pool, af_block_manager** out);
int af_bm_destroy(af_block_manager* bm);
int af_bm_attach_pool(af_block_manager* bm, void* base, const float* scales);
int af_bm_pool(const af_block_manager* bm, af_kv_pool* out);

/* allocate_block(): block id, or AF_ERR_POOL_EXHAUSTED (-1) (paged_kv_manager.h:105-107).
 * The new block has ref_count 1. */
int af_bm_allocate_block(af_block_manager* bm);
/* free_block(id) (paged_kv_manager.h:111): drops one reference; at zero the id
 * returns to the top of the free stack. */
int af_bm_free_block(af_block_manager* bm, int block_id);
int af_bm_num_free_blocks(const af_block_manager* bm);
/* ref_count of a block (0 when free), or AF_ERR_BAD_BLOCK. */
int af_bm_ref_count(const af_block_manager* bm, int block_id);

/* Sequences (PageTable = ordered block ids + last_block_fill). */
int af_bm_seq_create(af_block_manager* bm);              /* -> seq id */
int af_bm_seq_fork(af_block_manager* bm, int src_seq);   /* -> new seq id, every block ref+1 */
int af_bm_seq_free(af_block_manager* bm, int seq);       /* free_block on each block */
int af_bm_seq_len(const af_block_manager* bm, int seq);  /* tokens */
/* Writes up to max_ids block ids; returns the number of blocks. */
int af_bm_seq_table(const af_block_manager* bm, int seq, int32_t* ids, int max_ids,
                    int32_t* last_block_fill);
/* Plans one token append: a new block when the tail is full (or the table is
 * empty); copy-on-write when the tail is partial and shared (ref > 1): a new
 * block takes the tail's role, the caller copies rows [0, *cow_rows) from
 * *cow_src to *cow_dst for every layer (af_kv_copy_blocks), the old tail drops
 * one reference. Returns the new token's logical position; *slot = physical
 * row (block * block_size + offset). cow_* = -1 / 0 when no copy is needed.
 * On AF_ERR_POOL_EXHAUSTED nothing changes. */
int af_bm_seq_append(af_block_manager* bm, int seq, int64_t* slot, int32_t* cow_src,
                     int32_t* cow_dst, int32_t* cow_rows);
/* Appends n_tokens at once (prefill-style reservation, same rules per token).
 * Returns the first new position; copy-on-write of a shared tail is reported
 * as for af_bm_seq_append (at most one copy per call). */
int af_bm_seq_extend(af_block_manager* bm, int seq, int n_tokens, int32_t* cow_src,
                     int32_t* cow_dst, int32_t* cow_rows);
/* Physical row of logical token `pos` of `seq`, or a negative status. */
int64_t af_bm_seq_slot(const af_block_manager* bm, int seq, int pos);

/* Batched step planning for n sequences: one append each. Fills host arrays
 * slots[n], positions[n], copies[3*max_copies] (src, dst, rows) and *n_copies.
 * On failure no sequence is changed. */
int af_bm_plan_decode(af_block_manager* bm, const int32_t* seqs, int n, int64_t* slots,
                      int32_t* positions, int32_t* copies, int max_copies, int32_t* n_copies);
/* Copy-source holds, for a caller that plans several operations before it issues
 * their copies. A planned copy's source must keep its rows until the copy runs,
 * but a later free in the same plan (af_bm_seq_free, af_bm_free_block) may drop
 * its last reference, and the LIFO free list would hand it out again at once,
 * possibly as another copy's destination. af_bm_hold_copy_source(src) keeps a
 * referenced block off the free list when its references reach zero (a hold is
 * not a reference: the copy-on-write test ignores it); af_bm_release_copy_sources
 * drops every hold in the order taken and frees the unreferenced ones. The
 * scheduler (af_sched_step) holds its plan's sources and releases them before
 * returning. No reference counterpart (the reference declares no copy-on-write
 * bookkeeping: paged_kv_manager.h:51,61). hold: AF_OK or AF_ERR_BAD_BLOCK. */
int af_bm_hold_copy_source(af_block_manager* bm, int block_id);
int af_bm_release_copy_sources(af_block_manager* bm);
/* Block tables [n][max_blocks] (unused entries = 0) and lengths for n sequences. */
int af_bm_export_tables(const af_block_manager* bm, const int32_t* seqs, int n, int32_t* tables,
                        int max_blocks, int32_t* seq_lens);

/* ======================================================================== */
/* b3. Continuous-batching scheduler (ServerEngine::step)                    */
/* ======================================================================== */
/* Fills in the stub ServerEngine::step (src/experimental/server_arch/
 * server_engine.cu:55-68, server_engine.h:46-50: dequeue requests, build a
 * micro-batch, resolve PageTables for the batched attention, advance and retire)
 * over an af_block_manager; rules in include/server/scheduler.h. A step's plan is
 * read back with the af_sched_plan_* calls until the next af_sched_step. */
typedef struct af_scheduler af_scheduler;

/* max_step_tokens >= max_running >= 1, prefill_chunk >= 1, watermark >= 0. */
int af_sched_create(af_block_manager* bm, int max_running, int max_step_tokens,
                    int prefill_chunk, int watermark_blocks, af_scheduler** out);
int af_sched_destroy(af_scheduler* s);
/* FIFO; AF_ERR_INVALID_ARG if the request could never fit the pool alone. */
int af_sched_add_request(af_scheduler* s, int64_t id, int prompt_len, int max_new_tokens);
/* Prefix caching (no counterpart in the reference, whose server loop is a stub:
 * server_engine.cu:55-68; the fork it builds on is PageTable's "fork, bump
 * ref_counts", paged_kv_manager.h:61). A request whose first prefix_len
 * (< prompt_len) prompt tokens equal those of every request with the same
 * prefix_key: with the cache on, the first such request's prefill caches a fork
 * of its sequence at prefix_len, and later ones fork it and prefill only the
 * rest (their first append into a partial shared block is a CoW copy in the
 * plan). af_sched_set_prefix_cache sets the entry limit (0 = off, the default:
 * prefixes are then ignored); entries are evicted oldest-first when full and
 * before any preemption when the pool runs out. */
int af_sched_add_request_prefix(af_scheduler* s, int64_t id, int prompt_len, int max_new_tokens,
                                int64_t prefix_key, int prefix_len);
int af_sched_set_prefix_cache(af_scheduler* s, int max_entries);
int af_sched_clear_prefix_cache(af_scheduler* s);
/* This step's prefix events. counts (optional, int32[4]): requests admitted on
 * a cached prefix, prefixes cached, prefixes evicted, entries in the cache. The
 * arrays (optional) receive the request ids and the cached / evicted keys. */
int af_sched_plan_prefix(const af_scheduler* s, int32_t* counts, int64_t* hits, int64_t* cached,
                         int64_t* evicted);
/* Plans one step. counts (optional, int32[8]): decode sequences, prefill chunks,
 * prefill tokens, CoW copies, finished, preempted, running, waiting. */
int af_sched_step(af_scheduler* s, int32_t* counts);
/* Decode batch: request ids, sequence ids, slots, positions (the new token's
 * position; it attends position + 1 rows). Any pointer may be NULL. */
int af_sched_plan_decode(const af_scheduler* s, int64_t* requests, int32_t* seqs, int64_t* slots,
                         int32_t* positions);
/* Share groups of the decode batch (no counterpart in the reference): groups[i]
 * is the prefix-cache group of decode entry i (-1: none) and rows[i] the rows
 * [0, rows[i]) that every entry of that group holds with identical values (a
 * cached prefix's creator and every request admitted on it), so a caller may
 * attend them once per group with af_paged_attention_shared_prefix, using any
 * member's block table as the prefix table. Either pointer may be NULL. */
int af_sched_plan_decode_shared(const af_scheduler* s, int64_t* groups, int32_t* rows);
/* Prefill chunks: requests[i], chunks[5i..5i+4] = (seq, p0, n, offset, last);
 * slots / positions of every chunk token, chunk i at [offset, offset + n). */
int af_sched_plan_prefill(const af_scheduler* s, int64_t* requests, int32_t* chunks,
                          int64_t* slots, int32_t* positions);
/* CoW copies (src, dst, rows) to run (af_kv_copy_blocks) before the step's appends. */
int af_sched_plan_copies(const af_scheduler* s, int32_t* copies);
/* Requests retired at the start of the step, and requests preempted by it. */
int af_sched_plan_events(const af_scheduler* s, int64_t* finished, int64_t* preempted);

/* ======================================================================== */
/* b4. AtomFlow .bin weights (WeightLoader)                                 */
/* ======================================================================== */
/* The format of tools/quantize_weights.py:320-427 read by WeightLoader
 * (include/memory/weight_loader.h:23-130, src/core/engine.cu:97-148); layout in
 * include/memory/weight_loader.h. The file is mapped read-only; its payload (the
 * bytes after the 256-byte header) is uploaded as one block, so a tensor's
 * device address is dst + its payload offset. */
typedef struct af_weights af_weights;

/* AF_ERR_BAD_FILE when the file is missing, has no ATOM magic, an inconsistent
 * header, or fewer bytes than its layout needs. */
int af_weights_open(const char* path, af_weights** out);
int af_weights_close(af_weights* w);
/* Bytes of a file with header fields[9] (order of af_weights_header); 0 if the
 * header is inconsistent. */
size_t af_weights_layout_bytes(const int32_t* fields);
/* fields[9] = version, group_size, dim, hidden_dim, n_layers, n_heads,
 * n_kv_heads, vocab_size, max_seq_len. */
int af_weights_header(const af_weights* w, int32_t* fields);
size_t af_weights_payload_bytes(const af_weights* w);
/* Tensor kinds: 0 embed_tokens fp32 [V,D]; per layer 1 input_norm, 2 post_norm
 * fp32 [D]; 3 qkv E4M3 [D+2KV, D], 4 its fp16 scales; 5 o_proj [D,D], 6 scales;
 * 7 gate [F,D], 8 scales; 9 up [F,D], 10 scales; 11 down [D,F], 12 scales;
 * 13 final norm fp32 [D]; 14 lm_head fp16 [V,D]. layer = -1 for kinds 0, 13, 14.
 * offset: bytes from the payload start; dims[2] = rows, cols (cols 1 for vectors). */
int af_weights_tensor(const af_weights* w, int kind, int layer, int64_t* offset, int64_t* bytes,
                      int64_t* dims);
/* Copies the payload to device memory d_dst (dst_bytes >= payload bytes) through
 * pinned double buffers on `stream`; returns when the copy is complete. */
int af_weights_upload(const af_weights* w, void* d_dst, size_t dst_bytes, af_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* AF_KV_H_ */
