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
//  * D = X W^T on v_mfma_f32_32x32x16_f16. A = 32 tokens x 16 k of x, B = 16 k
//    x 32 weight rows (E4M3 -> fp16 in registers with v_cvt_scalef32_pk_f16_fp8
//    at scale 1, exact). Each lane loads 16 contiguous weight bytes per pair of
//    MFMAs; the pair's k order is permuted identically on both operands.
//  * D's column is the lane's weight row, so a group scale is one value per
//    lane: each group accumulates into a fresh fragment, then acc += scale * it.
//  * A workgroup is 4 waves = 128 weight rows (one head of the fused QKV) x one
//    of KS (<= 16) group-aligned slices of K of at most 512; the grid is row
//    blocks x KS x token tiles,
//    so every CU streams weights. The workgroup stages its x slice in LDS (rows
//    padded by 16 B against bank conflicts) and keeps 8 weight loads in flight
//    per wave.
//  * Slices are combined by the last workgroup of a row block to arrive (the
//    split-K protocol of the decode attention: agent-scope partial stores, one
//    relaxed agent-scope counter increment, re-armed by the last arrival), in
//    slice order, so results do not depend on timing. For the fused kernel the
//    rotation partners (d, d + 64) of the head are exchanged through LDS and
//    RoPE runs on the rounded fp16 projections.
#include <algorithm>
#include <cmath>

#include "af_common.h"
#include "af_device.h"

namespace af {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2v_t __attribute__((ext_vector_type(2)));
typedef float float16v_t __attribute__((ext_vector_type(16)));

constexpr int kBgWaves = 4;
constexpr int kBgThreads = 64 * kBgWaves;
constexpr int kBgTok = 32;          // tokens per token tile (one MFMA operand)
constexpr int kBgRows = 64;         // weight rows per workgroup: two 32-row tiles
constexpr int kBgDepth = 8;         // weight loads in flight per wave
constexpr int kBgCounterBytes = 64 * 1024;
constexpr int kBgMaxSliceK = 768;   // LDS: 32 x (768 + 8) fp16 + 10 KiB

struct BatchedArgs {
    const uint16_t* x;  // [m][x_stride] fp16
    int64_t x_stride;
    int m;
    const uint8_t* w;         // [n][k] E4M3
    const uint16_t* scales;   // [n][k / group_size] fp16
    int n, k, group_size, groups, slices;
    int slice_k;  // the widest slice's k extent
    uint16_t* y;  // [m][y_stride] fp16 (fused: qkv_out)
    int64_t y_stride;
    uint32_t* counters;  // [row blocks * token tiles]
    float* part;         // [row blocks * token tiles][slices][4 waves][64 lanes][16]
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
    // Dynamic LDS: the x slice [32 tokens][xs] fp16 (rows padded by 8 elements
    // against bank conflicts).
    extern __shared__ __align__(16) uint16_t s_x[];
    __shared__ float s_red[2][16][64];   // the second k-half's fragments
    __shared__ uint16_t s_y[16][64];     // fused: tile 1's rounded projections
    __shared__ int s_last;
    const int xs = a.slice_k + 8;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int tile = wave & 1, khalf = wave >> 1;  // waves 0,1: first k-half; 2,3: second
    const int col = lane & 31, hi = lane >> 5;
    const int blk = int(blockIdx.x), slice = int(blockIdx.y), ttile = int(blockIdx.z);
    const int t0 = ttile * kBgTok;
    const int mt = min(kBgTok, a.m - t0);   // tokens of this tile
    const int rmax = 4 * ((mt + 7) / 8);    // fragment registers holding them
    // The workgroup's tiles: plain, rows [64 blk, +64); fused (head_dim 128),
    // rows d and d + 64 of one head for d in [32 j, 32 j + 32).
    const int c0 = FUSED ? (blk >> 1) * 128 + 32 * (blk & 1) : blk * kBgRows;
    const int c = c0 + tile * (FUSED ? 64 : 32);
    const int nrow = min(c + col, a.n - 1);  // clamped loads

    const int g_lo = slice * a.groups / a.slices;
    const int g_hi = (slice + 1) * a.groups / a.slices;
    const int g_mid = g_lo + (g_hi - g_lo + 1) / 2;
    const int k0 = g_lo * a.group_size;                       // the slice
    const int kn = (g_hi - g_lo) * a.group_size;
    const int wg_lo = khalf ? g_mid : g_lo, wg_hi = khalf ? g_hi : g_mid;  // this wave
    const int iters = (wg_hi - wg_lo) * a.group_size / 32;
    const uint8_t* wrow = a.w + size_t(nrow) * a.k + size_t(wg_lo) * a.group_size + 16 * hi;

    // Weight loads first (they stream from HBM), then the x slice into LDS.
    uint4 wq[kBgDepth];
#pragma unroll
    for (int i = 0; i < kBgDepth; ++i)
        if (i < iters) wq[i] = *reinterpret_cast<const uint4*>(wrow + 32 * i);
    {
        const int chunks = kn / 8;  // 16-byte chunks per token row
        for (int e = tid; e < mt * chunks; e += kBgThreads) {
            const int t = e / chunks, ch = e % chunks;
            *reinterpret_cast<uint4*>(s_x + t * xs + 8 * ch) = *reinterpret_cast<const uint4*>(
                a.x + size_t(t0 + t) * a.x_stride + k0 + 8 * ch);
        }
    }
    __syncthreads();

    // Rows of s_x at or past mt are not written: their fragment rows are never
    // used (a D row depends only on its own A row).
    float16v_t acc, f;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = f[r] = 0.0f;
    const uint16_t* xl = s_x + col * xs + (wg_lo - g_lo) * a.group_size + 16 * hi;
    const int per_group = a.group_size / 32;
    for (int it0 = 0; it0 < iters; it0 += kBgDepth) {
#pragma unroll
        for (int i = 0; i < kBgDepth; ++i) {
            const int it = it0 + i;
            if (it < iters) {
                const uint4 wv = wq[i];
                if (it + kBgDepth < iters)  // refill the slot kBgDepth iterations ahead
                    wq[i] = *reinterpret_cast<const uint4*>(wrow + 32 * (it + kBgDepth));
                const half8_t xa = *reinterpret_cast<const half8_t*>(xl + 32 * it);
                const half8_t xb = *reinterpret_cast<const half8_t*>(xl + 32 * it + 8);
                f = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa, e4m3x8(wv.x, wv.y), f, 0, 0, 0);
                f = __builtin_amdgcn_mfma_f32_32x32x16_f16(xb, e4m3x8(wv.z, wv.w), f, 0, 0, 0);
                if ((it + 1) % per_group == 0) {  // group done: scale into the accumulator
                    const int g = wg_lo + it / per_group;
                    const float sc = h2f(a.scales[size_t(nrow) * a.groups + g]);
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        acc[r] = fmaf(sc, f[r], acc[r]);
                        f[r] = 0.0f;
                    }
                }
            }
        }
    }
    // The second k-half joins the first through LDS.
    if (khalf) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s_red[tile][r][lane] = acc[r];
    }
    __syncthreads();
    if (!khalf) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] += s_red[tile][r][lane];
    }

    // ---- slices: the last workgroup of the row block to arrive sums them -----
    const size_t rec = size_t(ttile) * gridDim.x + blk;
    if (!khalf) {
        float* my = a.part + ((rec * a.slices + slice) * 2 + tile) * 64 * 16 + lane * 16;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            if (r >= rmax) break;
            // (built as a float2: composing the 64-bit value from the two vector
            // elements with shifts compiled to one element stored twice)
            const float2 pr = make_float2(acc[r], acc[r + 1]);
            __hip_atomic_store(reinterpret_cast<uint64_t*>(my + r),
                               __builtin_bit_cast(uint64_t, pr), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        uint32_t* ctr = a.counters + rec;
        const uint32_t prev =
            __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev == uint32_t(a.slices - 1);
        if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;

    float v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = 0.0f;
    if (!khalf) {
        for (int sl = 0; sl < a.slices; ++sl) {
            const float* src = a.part + ((rec * a.slices + sl) * 2 + tile) * 64 * 16 + lane * 16;
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                if (r >= rmax) break;
                const uint64_t u = __hip_atomic_load(reinterpret_cast<const uint64_t*>(src + r),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                v[r] += __builtin_bit_cast(float, uint32_t(u));
                v[r + 1] += __builtin_bit_cast(float, uint32_t(u >> 32));
            }
        }
    }
    // Register r of lane l: token t0 + 8(r/4) + 4(l/32) + r%4, weight row c + l%32.
    if constexpr (!FUSED) {
        if (khalf) return;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + 8 * (r >> 2) + 4 * hi + (r & 3);
            if (t < a.m && c + col < a.n) a.y[size_t(t) * a.y_stride + c + col] = f2h(v[r]);
        }
    } else {
        if (tile == 1 && !khalf) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s_y[r][lane] = f2h(v[r]);
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
            const uint16_t y0 = f2h(v[r]), y1 = s_y[r][lane];
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

// Slices of K: the fewest whole-group slices of at most kBgMaxSliceK, at least
// 4 when K allows (so the grid streams from every CU).
int slices_for(int k, int group_size) {
    const int groups = k / group_size;
    const int per = std::max(1, kBgMaxSliceK / group_size);
    return std::min(groups, std::max(4, (groups + per - 1) / per));
}

size_t part_bytes(int m, int n, int k, int group_size) {
    const size_t recs = size_t((n + kBgRows - 1) / kBgRows) * ((m + kBgTok - 1) / kBgTok);
    return recs * slices_for(k, group_size) * 2 * 64 * 16 * sizeof(float);
}

int check_batched(const void* x, int64_t x_stride, int m, const uint8_t* w, const void* scales,
                  int n, int k, int group_size, const void* ws, size_t ws_bytes) {
    if (!x || !w || !scales || !ws || m < 0 || n <= 0 || k <= 0 || group_size <= 0)
        return AF_ERR_INVALID_ARG;
    if (k % 32 || group_size % 32 || k % group_size || group_size > kBgMaxSliceK)
        return AF_ERR_UNSUPPORTED;
    if (x_stride < k || x_stride % 8) return AF_ERR_INVALID_ARG;
    if (!aligned16(x) || !aligned16(w) || !aligned16(ws)) return AF_ERR_INVALID_ARG;
    const size_t recs = size_t((n + kBgRows - 1) / kBgRows) * ((m + kBgTok - 1) / kBgTok);
    if (recs * sizeof(uint32_t) > size_t(kBgCounterBytes)) return AF_ERR_UNSUPPORTED;
    if (ws_bytes < kBgCounterBytes + part_bytes(m, n, k, group_size)) return AF_ERR_WORKSPACE;
    return AF_OK;
}

void fill_common(BatchedArgs& a, const void* x, int64_t x_stride, int m, const uint8_t* w,
                 const void* scales, int n, int k, int group_size, void* ws) {
    a.x = static_cast<const uint16_t*>(x);
    a.x_stride = x_stride;
    a.m = m;
    a.w = w;
    a.scales = static_cast<const uint16_t*>(scales);
    a.n = n;
    a.k = k;
    a.group_size = group_size;
    a.groups = k / group_size;
    a.slices = slices_for(k, group_size);
    a.slice_k = (a.groups + a.slices - 1) / a.slices * group_size;
    a.counters = static_cast<uint32_t*>(ws);
    a.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kBgCounterBytes);
}

size_t lds_bytes(const BatchedArgs& a) { return size_t(kBgTok) * (a.slice_k + 8) * 2; }

}  // namespace
}  // namespace af

using namespace af;

extern "C" size_t af_gemm_batched_workspace_size(int m, int n, int k, int group_size) {
    if (m <= 0 || n <= 0 || k <= 0 || group_size <= 0 || k % group_size) return 0;
    return kBgCounterBytes + part_bytes(m, n, k, group_size);
}

extern "C" int af_gemm_batched_workspace_init(void* workspace, size_t workspace_bytes,
                                              af_stream_t stream) {
    if (!workspace || workspace_bytes < size_t(kBgCounterBytes)) return AF_ERR_INVALID_ARG;
    return fill_u32(workspace, 0u, kBgCounterBytes / 4, static_cast<hipStream_t>(stream));
}

extern "C" int af_w8a16_gemm_batched(const void* x, int64_t x_stride, int m, const uint8_t* weight,
                                     const void* scales, void* y, int64_t y_stride, int n, int k,
                                     int group_size, void* workspace, size_t workspace_bytes,
                                     af_stream_t stream) {
    if (int st = check_batched(x, x_stride, m, weight, scales, n, k, group_size, workspace,
                               workspace_bytes))
        return st;
    if (!y || y_stride < n) return AF_ERR_INVALID_ARG;
    if (m == 0) return AF_OK;
    BatchedArgs a{};
    fill_common(a, x, x_stride, m, weight, scales, n, k, group_size, workspace);
    a.y = static_cast<uint16_t*>(y);
    a.y_stride = y_stride;
    const dim3 grid((n + kBgRows - 1) / kBgRows, a.slices, (m + kBgTok - 1) / kBgTok);
    hipLaunchKernelGGL((w8a16_batched_kernel<false, false>), grid, dim3(kBgThreads),
                       lds_bytes(a), static_cast<hipStream_t>(stream), a);
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" int af_paged_qkv_rope_append(const void* x, int64_t x_stride, int m,
                                        const uint8_t* w_qkv, const void* scales, int k,
                                        int group_size, void* qkv_out, const af_kv_pool* pool,
                                        int layer, const int64_t* d_slots,
                                        const int32_t* d_positions, const float* cos_table,
                                        const float* sin_table, int max_pos, int n_q_heads,
                                        int32_t* d_status, void* workspace,
                                        size_t workspace_bytes, af_stream_t stream) {
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
    if (int st = check_batched(x, x_stride, m, w_qkv, scales, n, k, group_size, workspace,
                               workspace_bytes))
        return st;
    if (m == 0) return AF_OK;
    const size_t esz = fp8 ? 1 : 2;
    const int kv_dim = pool->n_kv_heads * hd;
    const size_t slab = size_t(pool->total_blocks) * pool->block_size * kv_dim * esz;
    uint8_t* base = static_cast<uint8_t*>(pool->base);
    BatchedArgs a{};
    fill_common(a, x, x_stride, m, w_qkv, scales, n, k, group_size, workspace);
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
    const dim3 grid(n / kBgRows, a.slices, (m + kBgTok - 1) / kBgTok);  // 2 per head
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t lds = lds_bytes(a);
    if (fp8)
        hipLaunchKernelGGL((w8a16_batched_kernel<true, true>), grid, dim3(kBgThreads), lds, s, a);
    else
        hipLaunchKernelGGL((w8a16_batched_kernel<true, false>), grid, dim3(kBgThreads), lds, s, a);
    AF_TRY_LAUNCH();
    return AF_OK;
}
