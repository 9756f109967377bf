// af_common.h — shared definitions for the gfx950 KV-cache kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "af_kv.h"

// Every kernel here is written for gfx950 (CDNA4) alone: wave64 reductions,
// its MFMA / transpose-load / FP8-convert forms, and the gfx9 memory-counter
// rules the split-K combine of decode_attention.hip depends on. Another device
// target must fail to build rather than compile into something subtly wrong.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "atomflow_amd kernels target gfx950 only: build with --offload-arch=gfx950"
#endif

#define AF_TRY_HIP(expr)                              \
    do {                                              \
        hipError_t af_e_ = (expr);                    \
        if (af_e_ != hipSuccess) return int(af_e_);   \
    } while (0)

// Launch-configuration errors surface here; execution faults surface at the
// next synchronising call, as with any HIP launch.
#define AF_TRY_LAUNCH()                               \
    do {                                              \
        hipError_t af_e_ = hipGetLastError();         \
        if (af_e_ != hipSuccess) return int(af_e_);   \
    } while (0)

namespace af {

constexpr int kWave = 64;
// Longest split grid; bounds the per-(sequence, head) partial buffers and lets
// the combine read every partial in one round of loads.
constexpr int kMaxSplits = 128;
// Target tokens per split of small launches: below this the partial (m, l, o[])
// traffic and the combine cost more than the split saves.
constexpr int kMinSpan = 64;
// Target tokens per split of batched launches (equal work per workgroup).
constexpr int kBatchSpan = 512;

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Split-K buffers of the decode-attention kernels. Layout of a workspace:
//   [0, kCounterBytes)           words [0, kMaxCounters): arrival counters, one
//                                per (sequence, KV head); words [kFlagBase,
//                                kFlagBase + kCombMaxGroups * kCombSplits):
//                                ready flags of the dedicated-combiner form, one
//                                per (sequence, KV head, split), then the poison
//                                word (set by a combiner that timed out); the
//                                last two
//                                words: the persistent form's item counters.
//                                Counters are zero between launches (each launch
//                                re-zeroes what it used)
//   [kCounterBytes, ...)         part_ml [batch][n_kv_heads][splits][2 * group]
//                                (group = n_q_heads / n_kv_heads: max..., sum...)
//   then                         part_o  [batch][n_kv_heads][splits][group * head_dim]
// The counter region has a fixed size and position and is zero between
// launches (each launch re-zeroes the counters it used), so one workspace
// serves launches of any batch / split count without re-initialisation.
constexpr size_t kCounterBytes = 64 * 1024;
constexpr int kMaxCounters = int(kCounterBytes / sizeof(uint32_t)) / 2;
constexpr int kFlagBase = kMaxCounters;
// Dedicated-combiner form: the most splits per (sequence, KV head), and the
// most (sequence, KV head) pairs of one launch (combiners are one workgroup
// each, dispatched after every split, and stay few enough that they could never
// hold every workgroup slot of the device).
constexpr int kCombSplits = 32;
constexpr int kCombMaxGroups = 16;
static_assert(kFlagBase + kCombMaxGroups * kCombSplits <= int(kCounterBytes / sizeof(uint32_t)),
              "ready flags exceed the counter region");
// Item and finished-workgroup counters of the persistent decode form (the last
// two words of the counter region).
constexpr int kItemCounter = int(kCounterBytes / sizeof(uint32_t)) - 2;
constexpr int kDoneCounter = kItemCounter + 1;
constexpr int kPoisonWord = kFlagBase + kCombMaxGroups * kCombSplits;
static_assert(kPoisonWord < kItemCounter, "counter words overlap");

struct AttnWorkspace {
    uint32_t* counters;
    uint32_t* flags;
    float* part_ml;
    float* part_o;
};

inline size_t attn_workspace_bytes(int batch, int n_q_heads, int head_dim, int num_splits) {
    const size_t pm = size_t(batch) * n_q_heads * num_splits * 2 * sizeof(float);
    const size_t po = size_t(batch) * n_q_heads * num_splits * head_dim * sizeof(float);
    return kCounterBytes + align_up(pm, 256) + align_up(po, 256);
}

inline AttnWorkspace attn_workspace_carve(void* base, int batch, int n_q_heads, int num_splits) {
    char* p = static_cast<char*>(base);
    AttnWorkspace w;
    w.counters = reinterpret_cast<uint32_t*>(p);
    w.flags = w.counters + kFlagBase;
    p += kCounterBytes;
    w.part_ml = reinterpret_cast<float*>(p);
    p += align_up(size_t(batch) * n_q_heads * num_splits * 2 * sizeof(float), 256);
    w.part_o = reinterpret_cast<float*>(p);
    return w;
}

// Number of compute units of the current device (cached per device).
int device_compute_units();

// Default split count: batched launches cover about kBatchSpan tokens per
// split; small ones about 3/4 of a workgroup per CU, each split at least
// kMinSpan tokens; at most kMaxSplits. `combiner`: the launch's shape can take
// the dedicated combiner (contiguous, head_dim 128, up to 4 query heads per KV
// head), which then leaves room for its combiner workgroups; default_splits
// assumes such a shape.
int default_splits_for(int max_seq_len, int batch, int n_kv_heads, bool combiner);
int default_splits(int max_seq_len, int batch, int n_kv_heads);
// Target tokens per split that goes with default_splits.
int default_span(int batch, int n_kv_heads);

// Fill kernel launcher shared by the runtime ABI and workspace init.
int fill_u32(void* dst, uint32_t value, size_t n_words, hipStream_t stream);

// Shared-prefix partials of paged decode attention: the matrix-core prefill
// kernel attends the decode queries of `batch` sequences (packed per KV head:
// the `group` Q heads of every sequence) over rows [0, prefix_len) of one block
// table, in key_splits key ranges, and writes split s of (sequence, KV head)
// to split-K record s (records rec_stride apart, the decode kernel's layout).
// head_dim 128. With cos_t the queries are rotated (RoPE) at positions[b].
struct PrefixPartialArgs {
    const uint16_t* q;  // row b at q + b * q_stride, Q head h at + h * 128
    int64_t q_stride;
    const uint8_t* k;   // the layer's K / V slabs
    const uint8_t* v;
    int64_t row_bytes;  // n_kv_heads * 128 * element size
    const float* scales;  // FP8 pools: this layer's [2][n_kv_heads]; NULL for fp16
    const int32_t* table;
    int bs_log2;
    int64_t total_blocks;  // block ids are clamped to [0, total_blocks)
    int prefix_len;
    int batch;
    int n_kv_heads;
    int group;
    int key_splits;
    int rec_stride;
    float* part_o;
    float* part_ml;
    const float* cos_t;
    const float* sin_t;
    const int32_t* positions;
    int max_pos;
};
// The single-token QKV projection + RoPE + KV append (gemv.hip), for the
// contiguous cache (rows = positions, max_rows = max_pos) and for one token of
// the paged pool (row = *d_slot, fp16 or FP8 with the layer's per-head scales).
enum { kQkvContiguous = 0, kQkvPagedFp16 = 1, kQkvPagedFp8 = 2 };
struct QkvSingleArgs {
    const uint8_t* w;        // [n_q + 2 n_kv heads][head_dim] x k E4M3 weights
    const uint16_t* x;       // k fp16 activations
    const uint16_t* scales;  // fp16 group scales
    int k, group_size;
    uint16_t* qkv;           // the projection (rotated Q and K)
    uint8_t* k_dst;          // K / V destination rows (fp16 or fp8 elements)
    uint8_t* v_dst;
    const float* cos_t;      // [max_pos][head_dim / 2]
    const float* sin_t;
    int pos_host;            // position when d_pos is NULL
    const int32_t* d_pos;
    int max_pos;
    const int64_t* d_slot;   // paged: the destination row
    int64_t max_rows;
    const float* k_scales;   // FP8: [n_kv_heads] each
    const float* v_scales;
    int n_q_heads, n_kv_heads, head_dim;
    int32_t* d_status;
};
void launch_qkv_single(const QkvSingleArgs& a, int dest, hipStream_t stream);

// Workgroups of the partial launch per key split.
int prefix_partial_tiles(int batch, int group, int n_kv_heads);
int launch_prefix_partials(const PrefixPartialArgs& p, hipStream_t stream);

}  // namespace af
