// gemm_batched.hip — the W8A16 projection for a batch of tokens on the gfx950
// matrix cores, and the paged serving step's fused QKV projection + RoPE +
// paged KV append.
//
//   y[m, n] = sum_k x[m, k] * e4m3(W[n, k]) * scale[n, k / group]
//
// is the reference's w8a16_gemv_kernel (src/kernel/qkv_gemm.cu:32-110) applied
// to each of M tokens: the reference engine decodes one token per step, a
// serving step one per sequence (the paged path's batch). fp32 accumulation,
// fp16 output; the fused form then rotates Q and K (rope.cu:30-45 arithmetic)
// and writes K and V to each token's slot of the paged pool, exactly as
// af_paged_rope_append does on the projection's output.
//
// Design (HBM-bound: one weight byte per 2*M flops; M <= 32 per token tile):
//  * D = X W^T on v_mfma_f32_32x32x16_f16. A = 32 tokens x 16 k of x (read
//    from L2, tokens past m read as zero), B = 16 k x 32 weight rows (E4M3 ->
//    fp16 in registers with v_cvt_scalef32_pk_f16_fp8 at scale 1, exact). A
//    lane loads 16 contiguous weight bytes per pair of MFMAs; the pair's k
//    order is permuted identically on both operands.
//  * D's column is the lane's weight row, so a group scale is one value per
//    lane: each group accumulates into a fresh fragment, then acc += scale * it.
//  * A workgroup is 16 waves: two 32-row tiles x eight group-aligned parts of
//    K. It owns its 64 rows' whole K, so no partial leaves the workgroup: the
//    parts are summed through LDS in a fixed tree (results do not depend on
//    timing) and the epilogue follows at once. Each wave keeps 8 weight loads
//    (8 KB) in flight, 128 KB per workgroup.
//  * For the fused kernel the two tiles are the rotation partners (d, d + 64)
//    of one head, exchanged through LDS; RoPE runs on the rounded fp16
//    projections.
#include <algorithm>
#include <cmath>

#include "af_common.h"
#include "af_device.h"

namespace af {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2v_t __attribute__((ext_vector_type(2)));
typedef float float16v_t __attribute__((ext_vector_type(16)));

constexpr int kBgParts = 8;                 // K parts per workgroup
constexpr int kBgWaves = 2 * kBgParts;       // two row tiles per part
constexpr int kBgThreads = 64 * kBgWaves;    // 1024
constexpr int kBgTok = 32;                   // tokens per token tile (one MFMA operand)
constexpr int kBgRows = 64;                  // weight rows per workgroup
constexpr int kBgDepth = 8;                  // weight loads in flight per wave

struct BatchedArgs {
    const uint16_t* x;  // [m][x_stride] fp16
    int64_t x_stride;
    int m;
    const uint8_t* w;         // [n][k] E4M3
    const uint16_t* scales;   // [n][k / group_size] fp16
    int n, k, group_size, groups;
    uint16_t* y;  // [m][y_stride] fp16 (fused: qkv_out)
    int64_t y_stride;
    // fused paged QKV only
    int n_q_heads, n_kv_heads, head_dim;
    const float* cos_t;
    const float* sin_t;
    int max_pos;
    const int32_t* d_positions;  // [m]
    const int64_t* d_slots;      // [m]
    int64_t max_rows;            // rows of one layer's K (or V) region
    uint8_t* k_dst;              // layer's K region (fp16 or fp8 elements)
    uint8_t* v_dst;
    const float* k_scales;  // fp8 pools: [n_kv_heads]
    const float* v_scales;
    int32_t* d_status;
};

// Eight E4M3 codes (two dwords) -> eight fp16 values, exact.
__device__ __forceinline__ half8_t e4m3x8(uint32_t lo, uint32_t hi) {
    const half2v_t a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(lo), 1.0f, false);
    const half2v_t b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(lo), 1.0f, true);
    const half2v_t c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(hi), 1.0f, false);
    const half2v_t d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(hi), 1.0f, true);
    return half8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// One rotation pair with the reference's separately rounded products.
__device__ __forceinline__ void rotate1(uint16_t x, uint16_t y, float c, float s, uint16_t& xo,
                                        uint16_t& yo) {
#pragma clang fp contract(off)
    const float xf = h2f(x), yf = h2f(y);
    const float xc = xf * c;
    const float ys = yf * s;
    const float xs = xf * s;
    const float yc = yf * c;
    xo = f2h(xc - ys);
    yo = f2h(xs + yc);
}

template <bool FUSED, bool FP8>
__global__ __launch_bounds__(kBgThreads) void w8a16_batched_kernel(const BatchedArgs a) {
    __shared__ float s_red[kBgParts][16][64];  // partial fragments, half the parts at a time
    __shared__ uint16_t s_y[16][64];           // fused: tile 1's rounded projections

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int tile = wave & 1, part = wave >> 1;
    const int col = lane & 31, hi = lane >> 5;
    const int blk = int(blockIdx.x), t0 = int(blockIdx.y) * kBgTok;
    // The workgroup's tiles: plain, rows [64 blk, +64); fused (head_dim 128),
    // rows d and d + 64 of one head for d in [32 j, 32 j + 32).
    const int c0 = FUSED ? (blk >> 1) * 128 + 32 * (blk & 1) : blk * kBgRows;
    const int c = c0 + tile * (FUSED ? 64 : 32);
    const int nrow = min(c + col, a.n - 1);  // clamped loads
    const int tok = t0 + col;
    const bool tok_live = tok < a.m;

    const int g_lo = part * a.groups / kBgParts, g_hi = (part + 1) * a.groups / kBgParts;
    const int iters = (g_hi - g_lo) * a.group_size / 32;
    const int kbase = g_lo * a.group_size + 16 * hi;
    const uint8_t* wrow = a.w + size_t(nrow) * a.k + kbase;
    const uint16_t* xr = a.x + size_t(tok_live ? tok : 0) * a.x_stride + kbase;

    uint4 wq[kBgDepth];
#pragma unroll
    for (int i = 0; i < kBgDepth; ++i)
        if (i < iters) wq[i] = *reinterpret_cast<const uint4*>(wrow + 32 * i);
    const uint4 zero4 = {0u, 0u, 0u, 0u};
    uint4 xa = zero4, xb = zero4;
    if (tok_live && iters > 0) {
        xa = *reinterpret_cast<const uint4*>(xr);
        xb = *reinterpret_cast<const uint4*>(xr + 8);
    }

    float16v_t acc, f;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = f[r] = 0.0f;
    const int per_group = a.group_size / 32;
    for (int it0 = 0; it0 < iters; it0 += kBgDepth) {
#pragma unroll
        for (int i = 0; i < kBgDepth; ++i) {
            const int it = it0 + i;
            if (it < iters) {
                const uint4 wv = wq[i];
                const half8_t x0 = __builtin_bit_cast(half8_t, xa);
                const half8_t x1 = __builtin_bit_cast(half8_t, xb);
                if (it + kBgDepth < iters)  // refill the slot kBgDepth iterations ahead
                    wq[i] = *reinterpret_cast<const uint4*>(wrow + 32 * (it + kBgDepth));
                if (tok_live && it + 1 < iters) {  // the next iteration's activations
                    xa = *reinterpret_cast<const uint4*>(xr + 32 * (it + 1));
                    xb = *reinterpret_cast<const uint4*>(xr + 32 * (it + 1) + 8);
                }
                f = __builtin_amdgcn_mfma_f32_32x32x16_f16(x0, e4m3x8(wv.x, wv.y), f, 0, 0, 0);
                f = __builtin_amdgcn_mfma_f32_32x32x16_f16(x1, e4m3x8(wv.z, wv.w), f, 0, 0, 0);
                if ((it + 1) % per_group == 0) {  // group done: scale into the accumulator
                    const float sc = h2f(a.scales[size_t(nrow) * a.groups + g_lo + it / per_group]);
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        acc[r] = fmaf(sc, f[r], acc[r]);
                        f[r] = 0.0f;
                    }
                }
            }
        }
    }

    // Sum the parts: a fixed tree through LDS (parts p and p + h, h = 4, 2, 1).
#pragma unroll
    for (int h = kBgParts / 2; h >= 1; h >>= 1) {
        if (part >= h && part < 2 * h) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s_red[(part - h) * 2 + tile][r][lane] = acc[r];
        }
        __syncthreads();
        if (part < h) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[r] += s_red[part * 2 + tile][r][lane];
        }
        __syncthreads();
    }

    // Register r of lane l: token t0 + 8(r/4) + 4(l/32) + r%4, weight row c + l%32.
    if constexpr (!FUSED) {
        if (part != 0) return;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + 8 * (r >> 2) + 4 * hi + (r & 3);
            if (t < a.m && c + col < a.n) a.y[size_t(t) * a.y_stride + c + col] = f2h(acc[r]);
        }
    } else {
        if (part == 0 && tile == 1) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s_y[r][lane] = f2h(acc[r]);
        }
        __syncthreads();
        if (wave != 0) return;  // wave 0 finishes the pairs (d, d + 64)
        const int hd = a.head_dim, half = hd / 2;
        const int head = c0 / hd;
        const int d = c0 % hd + col;
        const int kind = head < a.n_q_heads ? 0 : (head < a.n_q_heads + a.n_kv_heads ? 1 : 2);
        const int kh = head - a.n_q_heads - (kind == 2 ? a.n_kv_heads : 0);
        const int kv_dim = a.n_kv_heads * hd;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + 8 * (r >> 2) + 4 * hi + (r & 3);
            if (t >= a.m) continue;
            const uint16_t y0 = f2h(acc[r]), y1 = s_y[r][lane];
            uint16_t* yrow = a.y + size_t(t) * a.y_stride + size_t(head) * hd;
            const int pos = a.d_positions[t];
            const int64_t row = a.d_slots[t];
            if (pos < 0 || pos >= a.max_pos || row < 0 || row >= a.max_rows) {
                // nothing is rotated or appended for an out-of-range token
                yrow[d] = y0;
                yrow[d + half] = y1;
                if (a.d_status) *a.d_status = AF_ERR_OUT_OF_RANGE;
                continue;
            }
            uint16_t o0 = y0, o1 = y1;
            if (kind < 2)
                rotate1(y0, y1, a.cos_t[size_t(pos) * half + d], a.sin_t[size_t(pos) * half + d],
                        o0, o1);
            yrow[d] = o0;
            yrow[d + half] = o1;
            if (kind > 0) {
                const size_t e = size_t(row) * kv_dim + size_t(kh) * hd + d;
                uint8_t* base = kind == 1 ? a.k_dst : a.v_dst;
                if constexpr (FP8) {
                    const float sc = (kind == 1 ? a.k_scales : a.v_scales)[kh];
                    base[e] = uint8_t(quantize_fp8(o0, sc));
                    base[e + half] = uint8_t(quantize_fp8(o1, sc));
                } else {
                    reinterpret_cast<uint16_t*>(base)[e] = o0;
                    reinterpret_cast<uint16_t*>(base)[e + half] = o1;
                }
            }
        }
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_batched(const void* x, int64_t x_stride, int m, const uint8_t* w, const void* scales,
                  int n, int k, int group_size) {
    if (!x || !w || !scales || m < 0 || n <= 0 || k <= 0 || group_size <= 0)
        return AF_ERR_INVALID_ARG;
    if (k % 32 || group_size % 32 || k % group_size) return AF_ERR_UNSUPPORTED;
    if (x_stride < k || x_stride % 8) return AF_ERR_INVALID_ARG;
    if (!aligned16(x) || !aligned16(w)) return AF_ERR_INVALID_ARG;
    return AF_OK;
}

void fill_common(BatchedArgs& a, const void* x, int64_t x_stride, int m, const uint8_t* w,
                 const void* scales, int n, int k, int group_size) {
    a.x = static_cast<const uint16_t*>(x);
    a.x_stride = x_stride;
    a.m = m;
    a.w = w;
    a.scales = static_cast<const uint16_t*>(scales);
    a.n = n;
    a.k = k;
    a.group_size = group_size;
    a.groups = k / group_size;
}

}  // namespace
}  // namespace af

using namespace af;

extern "C" int af_w8a16_gemm_batched(const void* x, int64_t x_stride, int m, const uint8_t* weight,
                                     const void* scales, void* y, int64_t y_stride, int n, int k,
                                     int group_size, af_stream_t stream) {
    if (int st = check_batched(x, x_stride, m, weight, scales, n, k, group_size)) return st;
    if (!y || y_stride < n) return AF_ERR_INVALID_ARG;
    if (m == 0) return AF_OK;
    BatchedArgs a{};
    fill_common(a, x, x_stride, m, weight, scales, n, k, group_size);
    a.y = static_cast<uint16_t*>(y);
    a.y_stride = y_stride;
    const dim3 grid((n + kBgRows - 1) / kBgRows, (m + kBgTok - 1) / kBgTok);
    hipLaunchKernelGGL((w8a16_batched_kernel<false, false>), grid, dim3(kBgThreads), 0,
                       static_cast<hipStream_t>(stream), a);
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" int af_paged_qkv_rope_append(const void* x, int64_t x_stride, int m,
                                        const uint8_t* w_qkv, const void* scales, int k,
                                        int group_size, void* qkv_out, const af_kv_pool* pool,
                                        int layer, const int64_t* d_slots,
                                        const int32_t* d_positions, const float* cos_table,
                                        const float* sin_table, int max_pos, int n_q_heads,
                                        int32_t* d_status, af_stream_t stream) {
    if (!pool || !pool->base || !qkv_out || !d_slots || !d_positions || !cos_table ||
        !sin_table || max_pos <= 0 || n_q_heads <= 0)
        return AF_ERR_INVALID_ARG;
    if (layer < 0 || layer >= pool->n_layers) return AF_ERR_INVALID_ARG;
    const bool fp8 = pool->dtype == AF_KV_FP8_E4M3;
    if (!fp8 && pool->dtype != AF_KV_FP16) return AF_ERR_UNSUPPORTED;
    if (fp8 && !pool->scales) return AF_ERR_INVALID_ARG;
    if (pool->n_kv_heads <= 0) return AF_ERR_INVALID_ARG;
    const int hd = pool->head_dim;
    if (hd != 128) return AF_ERR_UNSUPPORTED;  // a workgroup's tiles are d and d + 64
    const int n = (n_q_heads + 2 * pool->n_kv_heads) * hd;
    if (int st = check_batched(x, x_stride, m, w_qkv, scales, n, k, group_size)) return st;
    if (m == 0) return AF_OK;
    const size_t esz = fp8 ? 1 : 2;
    const int kv_dim = pool->n_kv_heads * hd;
    const size_t slab = size_t(pool->total_blocks) * pool->block_size * kv_dim * esz;
    uint8_t* base = static_cast<uint8_t*>(pool->base);
    BatchedArgs a{};
    fill_common(a, x, x_stride, m, w_qkv, scales, n, k, group_size);
    a.y = static_cast<uint16_t*>(qkv_out);
    a.y_stride = n;
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = pool->n_kv_heads;
    a.head_dim = hd;
    a.cos_t = cos_table;
    a.sin_t = sin_table;
    a.max_pos = max_pos;
    a.d_positions = d_positions;
    a.d_slots = d_slots;
    a.max_rows = int64_t(pool->total_blocks) * pool->block_size;
    a.k_dst = base + size_t(2 * layer) * slab;
    a.v_dst = base + size_t(2 * layer + 1) * slab;
    if (fp8) {
        a.k_scales = pool->scales + size_t(layer) * 2 * pool->n_kv_heads;
        a.v_scales = a.k_scales + pool->n_kv_heads;
    }
    a.d_status = d_status;
    const dim3 grid(n / kBgRows, (m + kBgTok - 1) / kBgTok);  // two per head
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (fp8)
        hipLaunchKernelGGL((w8a16_batched_kernel<true, true>), grid, dim3(kBgThreads), 0, s, a);
    else
        hipLaunchKernelGGL((w8a16_batched_kernel<true, false>), grid, dim3(kBgThreads), 0, s, a);
    AF_TRY_LAUNCH();
    return AF_OK;
}
