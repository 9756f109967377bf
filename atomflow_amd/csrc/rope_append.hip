// rope_append.hip — RoPE table, RoPE, KV write and the fused RoPE+append
// kernels for gfx950.
//
// Numerics follow the reference bit for bit: each rotated element is
// (x*c - y*s) or (x*s + y*c) with separately rounded fp32 products and sum
// (src/kernel/rope.cu:34-35,43-44), then one fp32 -> fp16 round-to-nearest-even
// (the `(T)` cast). rope_rotate (af_device.h) disables FMA contraction, which
// would change the last bit.
#include <cmath>
#include <cstring>
#include <vector>

#include "af_common.h"
#include "af_device.h"

namespace af {
namespace {

// One rotation of four (x, y) pairs: pairs d..d+3 of a head.
__device__ __forceinline__ void rotate4(const uint16_t (&x)[4], const uint16_t (&y)[4],
                                        const float (&c)[4], const float (&s)[4],
                                        uint16_t (&xo)[4], uint16_t (&yo)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) rope_rotate(x[i], y[i], c[i], s[i], xo[i], yo[i]);
}

__device__ __forceinline__ void load4h(const uint16_t* p, uint16_t (&v)[4]) {
    const uint2 w = *reinterpret_cast<const uint2*>(p);
    v[0] = uint16_t(w.x & 0xffffu);
    v[1] = uint16_t(w.x >> 16);
    v[2] = uint16_t(w.y & 0xffffu);
    v[3] = uint16_t(w.y >> 16);
}
__device__ __forceinline__ void store4h(uint16_t* p, const uint16_t (&v)[4]) {
    uint2 w;
    w.x = uint32_t(v[0]) | (uint32_t(v[1]) << 16);
    w.y = uint32_t(v[2]) | (uint32_t(v[3]) << 16);
    *reinterpret_cast<uint2*>(p) = w;
}
__device__ __forceinline__ void load4f(const float* p, float (&v)[4]) {
    const float4 w = *reinterpret_cast<const float4*>(p);
    v[0] = w.x;
    v[1] = w.y;
    v[2] = w.z;
    v[3] = w.w;
}

// ---- reference-shaped RoPE: src/kernel/rope.cu:11-46 ------------------------
// grid = seq_len tokens; each thread rotates 4 pairs of one head.
__global__ void rope_rows_kernel(uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                                 const float* __restrict__ cos_cache,
                                 const float* __restrict__ sin_cache, int kv_heads, int q_heads,
                                 int head_dim) {
    const int p = blockIdx.x;
    const int half = head_dim / 2;
    const int quads = half / 4;
    const int items = (q_heads + kv_heads) * quads;
    for (int it = threadIdx.x; it < items; it += blockDim.x) {
        const int head = it / quads;
        const int d0 = (it % quads) * 4;
        uint16_t* base = head < q_heads
                             ? q + (size_t(p) * q_heads + head) * head_dim
                             : k + (size_t(p) * kv_heads + (head - q_heads)) * head_dim;
        uint16_t x[4], y[4], xo[4], yo[4];
        float c[4], s[4];
        load4h(base + d0, x);
        load4h(base + half + d0, y);
        load4f(cos_cache + size_t(p) * half + d0, c);
        load4f(sin_cache + size_t(p) * half + d0, s);
        rotate4(x, y, c, s, xo, yo);
        store4h(base + d0, xo);
        store4h(base + half + d0, yo);
    }
}

// ---- reference-shaped KV write: src/kernel/helpers.cu:126-139 ----------------
__global__ void write_kv_kernel(const uint16_t* __restrict__ qkv_out, uint16_t* __restrict__ k_dst,
                                uint16_t* __restrict__ v_dst, int q_dim, int kv_dim) {
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i >= kv_dim) return;
    *reinterpret_cast<uint4*>(k_dst + i) = *reinterpret_cast<const uint4*>(qkv_out + q_dim + i);
    *reinterpret_cast<uint4*>(v_dst + i) =
        *reinterpret_cast<const uint4*>(qkv_out + q_dim + kv_dim + i);
}

// ---- fused RoPE + append ------------------------------------------------------
// One workgroup per sequence. Work items: (n_q_heads + n_kv_heads) * head_dim/8
// rotations of four pairs, then kv_dim/8 V copies of eight elements. Q and K
// are rotated in place in qkv_out; rotated K and V go to row `row` of the
// destination (contiguous cache: row = position; paged pool: row = slot).
struct RopeAppendArgs {
    uint16_t* qkv;
    int64_t qkv_stride;  // elements between sequences
    const float* cos_t;
    const float* sin_t;
    int32_t max_pos;        // rows in the RoPE table
    const int32_t* d_pos;   // [batch] positions, or NULL -> pos_host
    int32_t pos_host;
    int32_t d_pos_shared;   // 1: every row reads d_pos[0]
    int32_t pos_inc;        // row b adds b * pos_inc (1 for the rows of a prompt chunk)
    const int64_t* d_slots; // [batch] destination rows, or NULL -> row = position
    int64_t max_rows;       // rows in the destination
    uint8_t* k_dst;         // destination bases (fp16 or fp8 elements)
    uint8_t* v_dst;
    const float* k_scales;  // fp8: [n_kv_heads]
    const float* v_scales;
    int32_t n_q_heads;
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t* d_status;
};

template <bool FP8>
__global__ __launch_bounds__(256) void rope_append_kernel(const RopeAppendArgs a) {
    const int b = blockIdx.x;
    const int pos = (a.d_pos ? a.d_pos[a.d_pos_shared ? 0 : b] : a.pos_host) + a.pos_inc * b;
    const int64_t row = a.d_slots ? a.d_slots[b] : int64_t(pos);
    if (pos < 0 || pos >= a.max_pos || row < 0 || row >= a.max_rows) {
        if (threadIdx.x == 0 && a.d_status) *a.d_status = AF_ERR_OUT_OF_RANGE;
        return;  // nothing is written for an out-of-range append
    }
    const int hd = a.head_dim;
    const int half = hd / 2;
    const int quads = half / 4;
    const int q_dim = a.n_q_heads * hd;
    const int kv_dim = a.n_kv_heads * hd;
    uint16_t* qkv = a.qkv + size_t(b) * a.qkv_stride;
    const float* crow = a.cos_t + size_t(pos) * half;
    const float* srow = a.sin_t + size_t(pos) * half;
    const int rot_items = (a.n_q_heads + a.n_kv_heads) * quads;
    const int v_items = kv_dim / 8;
    for (int it = threadIdx.x; it < rot_items + v_items; it += blockDim.x) {
        if (it < rot_items) {
            const int head = it / quads;
            const int d0 = (it % quads) * 4;
            const bool is_k = head >= a.n_q_heads;
            uint16_t* base = qkv + size_t(head) * hd;  // K heads follow Q heads in the row
            uint16_t x[4], y[4], xo[4], yo[4];
            float c[4], s[4];
            load4h(base + d0, x);
            load4h(base + half + d0, y);
            load4f(crow + d0, c);
            load4f(srow + d0, s);
            rotate4(x, y, c, s, xo, yo);
            store4h(base + d0, xo);
            store4h(base + half + d0, yo);
            if (is_k) {
                const int kh = head - a.n_q_heads;
                const size_t col = size_t(kh) * hd + d0;
                if constexpr (FP8) {
                    const float sc = a.k_scales[kh];
                    uint8_t* dst = a.k_dst + size_t(row) * kv_dim + col;
                    uint32_t wx = 0, wy = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        wx |= quantize_fp8(xo[i], sc) << (8 * i);
                        wy |= quantize_fp8(yo[i], sc) << (8 * i);
                    }
                    *reinterpret_cast<uint32_t*>(dst) = wx;
                    *reinterpret_cast<uint32_t*>(dst + half) = wy;
                } else {
                    uint16_t* dst = reinterpret_cast<uint16_t*>(a.k_dst) + size_t(row) * kv_dim + col;
                    store4h(dst, xo);
                    store4h(dst + half, yo);
                }
            }
        } else {
            const int e = (it - rot_items) * 8;
            const uint4 v = *reinterpret_cast<const uint4*>(qkv + q_dim + kv_dim + e);
            if constexpr (FP8) {
                const float sc = a.v_scales[e / hd];
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
                uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    lo |= quantize_fp8(uint16_t(w[i / 2] >> (16 * (i % 2))), sc) << (8 * i);
                    hi |= quantize_fp8(uint16_t(w[2 + i / 2] >> (16 * (i % 2))), sc) << (8 * i);
                }
                uint2 o;
                o.x = lo;
                o.y = hi;
                *reinterpret_cast<uint2*>(a.v_dst + size_t(row) * kv_dim + e) = o;
            } else {
                *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(a.v_dst) +
                                          size_t(row) * kv_dim + e) = v;
            }
        }
    }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace af

using namespace af;

// ---- a1 -----------------------------------------------------------------------
// build_rope_cache (src/kernel/helpers.cu:94-113): float powf/cosf/sinf on the
// host, then a copy to the device. Computed on the host so the table holds the
// same bytes as the reference's host-built table.
extern "C" int af_rope_table_host(float* h_cos, float* h_sin, int max_seq, int head_dim,
                                  float base) {
    if (!h_cos || !h_sin || max_seq <= 0 || head_dim <= 0 || (head_dim % 2)) return AF_ERR_INVALID_ARG;
    const int half_dim = head_dim / 2;
    for (int s = 0; s < max_seq; ++s) {
        for (int i = 0; i < half_dim; ++i) {
            const float expo = 2.0f * float(i) / float(head_dim);
            const float theta = float(s) / std::pow(base, expo);
            h_cos[size_t(s) * half_dim + i] = std::cos(theta);
            h_sin[size_t(s) * half_dim + i] = std::sin(theta);
        }
    }
    return AF_OK;
}

extern "C" int af_rope_table_build(float* d_cos, float* d_sin, int max_seq, int head_dim,
                                   float base, af_stream_t stream) {
    if (!d_cos || !d_sin || max_seq <= 0 || head_dim <= 0 || (head_dim % 2)) return AF_ERR_INVALID_ARG;
    const size_t n = size_t(max_seq) * (head_dim / 2);
    std::vector<float> hc(n), hs(n);
    int st = af_rope_table_host(hc.data(), hs.data(), max_seq, head_dim, base);
    if (st) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    AF_TRY_HIP(hipMemcpyAsync(d_cos, hc.data(), n * sizeof(float), hipMemcpyHostToDevice, s));
    AF_TRY_HIP(hipMemcpyAsync(d_sin, hs.data(), n * sizeof(float), hipMemcpyHostToDevice, s));
    AF_TRY_HIP(hipStreamSynchronize(s));  // host staging buffers die on return
    return AF_OK;
}

// ---- a2 -----------------------------------------------------------------------
extern "C" int af_rope(void* q, void* k, const float* cos_cache, const float* sin_cache,
                       int seq_len, int kv_head_num, int q_head_num, int head_dim,
                       af_stream_t stream) {
    if (!q || !k || !cos_cache || !sin_cache || seq_len < 0 || kv_head_num <= 0 ||
        q_head_num <= 0 || head_dim <= 0 || head_dim % 8)
        return AF_ERR_INVALID_ARG;
    if (!aligned16(q) || !aligned16(k) || !aligned16(cos_cache) || !aligned16(sin_cache))
        return AF_ERR_INVALID_ARG;
    if (seq_len == 0) return AF_OK;
    hipLaunchKernelGGL(rope_rows_kernel, dim3(seq_len), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<uint16_t*>(q),
                       static_cast<uint16_t*>(k), cos_cache, sin_cache, kv_head_num, q_head_num,
                       head_dim);
    AF_TRY_LAUNCH();
    return AF_OK;
}

// ---- a3 -----------------------------------------------------------------------
extern "C" int af_write_kv_cache(const void* qkv_out, void* k_cache, void* v_cache,
                                 int current_pos, int max_seq, int q_dim, int kv_dim,
                                 af_stream_t stream) {
    if (!qkv_out || !k_cache || !v_cache || q_dim <= 0 || kv_dim <= 0 || kv_dim % 8 || q_dim % 8)
        return AF_ERR_INVALID_ARG;
    if (!aligned16(qkv_out) || !aligned16(k_cache) || !aligned16(v_cache)) return AF_ERR_INVALID_ARG;
    if (current_pos < 0 || current_pos >= max_seq) return AF_ERR_OUT_OF_RANGE;
    uint16_t* kd = static_cast<uint16_t*>(k_cache) + size_t(current_pos) * kv_dim;
    uint16_t* vd = static_cast<uint16_t*>(v_cache) + size_t(current_pos) * kv_dim;
    const int threads = 128;
    const int blocks = ceil_div(kv_dim / 8, threads);
    hipLaunchKernelGGL(write_kv_kernel, dim3(blocks), dim3(threads), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(qkv_out), kd,
                       vd, q_dim, kv_dim);
    AF_TRY_LAUNCH();
    return AF_OK;
}

// ---- a2+a3 fused --------------------------------------------------------------
extern "C" int af_rope_append(void* qkv_out, void* k_cache, void* v_cache, const float* cos_table,
                              const float* sin_table, int pos, const int32_t* d_pos, int max_seq,
                              int n_q_heads, int n_kv_heads, int head_dim, int32_t* d_status,
                              af_stream_t stream) {
    if (!qkv_out || !k_cache || !v_cache || !cos_table || !sin_table || max_seq <= 0 ||
        n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 8)
        return AF_ERR_INVALID_ARG;
    if (!aligned16(qkv_out) || !aligned16(k_cache) || !aligned16(v_cache) ||
        !aligned16(cos_table) || !aligned16(sin_table))
        return AF_ERR_INVALID_ARG;
    if (!d_pos && (pos < 0 || pos >= max_seq)) return AF_ERR_OUT_OF_RANGE;
    RopeAppendArgs a{};
    a.qkv = static_cast<uint16_t*>(qkv_out);
    a.qkv_stride = int64_t(n_q_heads + 2 * n_kv_heads) * head_dim;
    a.cos_t = cos_table;
    a.sin_t = sin_table;
    a.max_pos = max_seq;  // the table covers every cache row
    a.d_pos = d_pos;
    a.pos_host = pos;
    a.d_slots = nullptr;
    a.max_rows = max_seq;
    a.k_dst = static_cast<uint8_t*>(k_cache);
    a.v_dst = static_cast<uint8_t*>(v_cache);
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.d_status = d_status;
    hipLaunchKernelGGL(rope_append_kernel<false>, dim3(1), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a);
    AF_TRY_LAUNCH();
    return AF_OK;
}

// ---- b2: multi-token append ----------------------------------------------------
extern "C" int af_prefill_rope_append(void* qkv_out, int n, void* k_cache, void* v_cache,
                                      const float* cos_table, const float* sin_table, int p0,
                                      const int32_t* d_p0, int max_seq, int n_q_heads,
                                      int n_kv_heads, int head_dim, int32_t* d_status,
                                      af_stream_t stream) {
    if (!qkv_out || !k_cache || !v_cache || !cos_table || !sin_table || n < 0 || max_seq <= 0 ||
        n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 8)
        return AF_ERR_INVALID_ARG;
    if (!aligned16(qkv_out) || !aligned16(k_cache) || !aligned16(v_cache) ||
        !aligned16(cos_table) || !aligned16(sin_table))
        return AF_ERR_INVALID_ARG;
    if (!d_p0 && (p0 < 0 || int64_t(p0) + n > max_seq)) return AF_ERR_OUT_OF_RANGE;
    if (n == 0) return AF_OK;
    RopeAppendArgs a{};
    a.qkv = static_cast<uint16_t*>(qkv_out);
    a.qkv_stride = int64_t(n_q_heads + 2 * n_kv_heads) * head_dim;
    a.cos_t = cos_table;
    a.sin_t = sin_table;
    a.max_pos = max_seq;
    a.d_pos = d_p0;
    a.pos_host = p0;
    a.d_pos_shared = 1;
    a.pos_inc = 1;
    a.d_slots = nullptr;
    a.max_rows = max_seq;
    a.k_dst = static_cast<uint8_t*>(k_cache);
    a.v_dst = static_cast<uint8_t*>(v_cache);
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.d_status = d_status;
    hipLaunchKernelGGL(rope_append_kernel<false>, dim3(n), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a);
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" size_t af_kv_pool_bytes(const af_kv_pool* p) {
    if (!p) return 0;
    const size_t esz = p->dtype == AF_KV_FP8_E4M3 ? 1 : 2;
    return size_t(p->n_layers) * 2 * size_t(p->total_blocks) * p->block_size * p->n_kv_heads *
           p->head_dim * esz;
}

extern "C" int af_paged_rope_append(void* qkv_out, int batch, const af_kv_pool* pool, int layer,
                                    const int64_t* d_slots, const int32_t* d_positions,
                                    const float* cos_table, const float* sin_table, int max_pos,
                                    int n_q_heads, af_stream_t stream) {
    if (!qkv_out || !pool || !pool->base || !d_slots || !d_positions || !cos_table ||
        !sin_table || batch < 0 || max_pos <= 0 || n_q_heads <= 0)
        return AF_ERR_INVALID_ARG;
    if (layer < 0 || layer >= pool->n_layers) return AF_ERR_INVALID_ARG;
    if (pool->flags & ~AF_KV_POOL_SHARED_BLOCKS) return AF_ERR_INVALID_ARG;
    const bool fp8 = pool->dtype == AF_KV_FP8_E4M3;
    if (!fp8 && pool->dtype != AF_KV_FP16) return AF_ERR_UNSUPPORTED;
    if (fp8 && !pool->scales) return AF_ERR_INVALID_ARG;
    const int hd = pool->head_dim;
    if (hd <= 0 || hd % 8 || pool->n_kv_heads <= 0) return AF_ERR_INVALID_ARG;
    if (!aligned16(qkv_out) || !aligned16(pool->base) || !aligned16(cos_table) ||
        !aligned16(sin_table))
        return AF_ERR_INVALID_ARG;
    if (batch == 0) return AF_OK;
    const size_t esz = fp8 ? 1 : 2;
    const int kv_dim = pool->n_kv_heads * hd;
    const size_t slab = size_t(pool->total_blocks) * pool->block_size * kv_dim * esz;
    uint8_t* base = static_cast<uint8_t*>(pool->base);
    RopeAppendArgs a{};
    a.qkv = static_cast<uint16_t*>(qkv_out);
    a.qkv_stride = int64_t(n_q_heads + 2 * pool->n_kv_heads) * hd;
    a.cos_t = cos_table;
    a.sin_t = sin_table;
    a.max_pos = max_pos;
    a.d_pos = d_positions;
    a.pos_host = 0;
    a.d_slots = d_slots;
    a.max_rows = int64_t(pool->total_blocks) * pool->block_size;
    a.k_dst = base + size_t(2 * layer) * slab;
    a.v_dst = base + size_t(2 * layer + 1) * slab;
    if (fp8) {
        a.k_scales = pool->scales + size_t(layer) * 2 * pool->n_kv_heads;
        a.v_scales = a.k_scales + pool->n_kv_heads;
    }
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = pool->n_kv_heads;
    a.head_dim = hd;
    a.d_status = nullptr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (fp8)
        hipLaunchKernelGGL(rope_append_kernel<true>, dim3(batch), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(rope_append_kernel<false>, dim3(batch), dim3(256), 0, s, a);
    AF_TRY_LAUNCH();
    return AF_OK;
}
