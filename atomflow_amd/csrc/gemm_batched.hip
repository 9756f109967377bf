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
// Design (HBM-bound: one weight byte per 2*M flops; M <= 32 per launch tile):
//  * D = X W^T on v_mfma_f32_16x16x32_f16: A = 16 tokens x 32 k of x (read
//    from L2; rows past m repeat row m-1 and are not stored), B = 32 k x 16
//    weight rows (E4M3 -> fp16 in registers with v_cvt_scalef32_pk_f16_fp8 at
//    scale 1, exact). With group sizes that are multiples of 64, a lane loads 16 contiguous weight
//    bytes per pair of MFMAs and the pair's k order is permuted identically on
//    both operands; otherwise 8 bytes per MFMA.
//  * D's column is the lane's weight row, so a group scale is one value per
//    lane: each group accumulates into a fresh fragment, then acc += scale * it.
//  * A workgroup is 8 waves over 16 weight rows: wave p owns the p-th
//    group-aligned part of K, so each workgroup owns its rows' whole K and no
//    partial leaves it. The parts are summed through LDS in a fixed order
//    (results do not depend on timing). 16-row workgroups spread the weights
//    over every CU (320 workgroups for the 5120-row QKV projection); up to 32
//    tokens (two token tiles) share each weight load.
//  * For the fused kernel the 16 columns are 8 head dims d and their rotation
//    partners d + 64, so a pair sits in lanes l and l ^ 8 of a 16-lane row;
//    RoPE runs on the rounded fp16 projections.
#include <algorithm>
#include <cmath>

#include "af_common.h"
#include "af_device.h"

namespace af {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2v_t __attribute__((ext_vector_type(2)));

typedef float float4v_t __attribute__((ext_vector_type(4)));

constexpr int kBgParts = 8;               // K parts = waves per workgroup
constexpr int kBgThreads = 64 * kBgParts;  // 512
constexpr int kBgRows = 16;               // weight rows per workgroup (one MFMA column tile)
constexpr int kBgTile = 16;               // tokens per token tile (one MFMA row tile)

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

// Weight bytes of one lane for one chunk: 16 (KC = 64) or 8 (KC = 32).
template <int KC>
struct WChunk {
    uint4 v;
};
template <>
struct WChunk<32> {
    uint2 v;
};

// TT token tiles x KC k per chunk; DEPTH chunks in flight per wave.
template <bool FUSED, bool FP8, int TT, int KC>
__global__ __launch_bounds__(kBgThreads, 4) void w8a16_batched_kernel(const BatchedArgs a) {
    constexpr int DEPTH = TT == 1 ? 6 : (KC == 64 ? 2 : 3);  // <= 128 VGPRs: two workgroups per CU
    constexpr int XV = KC / 32;  // 16-byte x loads per token tile per chunk
    __shared__ float s_red[kBgParts][TT * 4][64];
    // KC = 64: each wave's x chunk goes through LDS (see below), 2 KB per token tile.
    __shared__ uint4 s_x[KC == 64 ? kBgParts : 1][TT][2][64];
    __shared__ int32_t s_pos[FUSED ? kBgTile * TT : 1];
    __shared__ int64_t s_slot[FUSED ? kBgTile * TT : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int part = tid >> 6;
    const int j = lane & 15, sub = lane >> 4;  // MFMA column / row index, k sub-block
    const int blk = int(blockIdx.x), t0 = int(blockIdx.y) * kBgTile * TT;
    // The workgroup's 16 weight rows: plain, [16 blk, +16); fused (head_dim 128),
    // dims d0 .. d0+7 of head blk/8 (d0 = 8 (blk % 8)) and their partners d + 64.
    int row;
    if constexpr (FUSED)
        row = (blk >> 3) * 128 + (blk & 7) * 8 + (j & 7) + (j >> 3) * 64;
    else
        row = blk * kBgRows + j;
    const int nrow = min(row, a.n - 1);  // clamped loads

    const int g_lo = part * a.groups / kBgParts, g_hi = (part + 1) * a.groups / kBgParts;
    const int chunks = (g_hi - g_lo) * a.group_size / KC;
    const int per_group = a.group_size / KC;
    const int kbase = g_lo * a.group_size + sub * (KC / 4);  // this lane's first k in a chunk
    const uint8_t* wrow = a.w + size_t(nrow) * a.k + kbase;
    // Token rows past m load row m-1 instead: an MFMA output row depends only on
    // its own A row, and those rows' outputs are never written. (Loading zeros
    // there instead made the compiler select between the x address and a
    // scratch copy of zero, i.e. flat loads, at twice the kernel's time.)
    //
    // KC = 64: x is loaded row-contiguous, not in the MFMA operand layout (which
    // gives the 16 lanes of a k block 16 different token rows, so each load
    // instruction would touch 16 half-used cache lines). Load v of a token tile
    // covers tokens 8v .. 8v+7, one 128-byte line (64 k) per 8 lanes: lane l
    // fetches piece p = (l % 8) ^ ((r / 2) % 8) of token r = 8v + l / 8. The chunk
    // is written to the wave's LDS stage in lane order and read back in operand
    // order; the XOR makes the read of the 16 lanes of a k block hit 16 distinct
    // 16-byte bank groups.
    const uint16_t* xr[TT][KC / 32];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        if constexpr (KC == 64) {
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                const int r = 8 * v + (lane >> 3);
                const int piece = (lane & 7) ^ ((r >> 1) & 7);
                const int tok = min(t0 + kBgTile * tt + r, a.m - 1);
                xr[tt][v] = a.x + size_t(tok) * a.x_stride + g_lo * a.group_size + 8 * piece;
            }
        } else {
            const int tok = min(t0 + kBgTile * tt + j, a.m - 1);
            xr[tt][0] = a.x + size_t(tok) * a.x_stride + kbase;
        }
    }

    WChunk<KC> wq[DEPTH];
    uint4 xq[DEPTH][TT][XV];
    uint16_t sq[DEPTH];  // the group scale of each chunk in flight
    const uint16_t* srow = a.scales + size_t(nrow) * a.groups + g_lo;
    auto issue = [&](int slot, int c) __attribute__((always_inline)) {
        sq[slot] = srow[c / per_group];
        if constexpr (KC == 64)
            wq[slot].v = *reinterpret_cast<const uint4*>(wrow + size_t(c) * KC);
        else
            wq[slot].v = *reinterpret_cast<const uint2*>(wrow + size_t(c) * KC);
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int v = 0; v < XV; ++v)
                xq[slot][tt][v] = *reinterpret_cast<const uint4*>(xr[tt][v] + size_t(c) * KC);
    };
#pragma unroll
    for (int i = 0; i < DEPTH; ++i)
        if (i < chunks) issue(i, i);
    if constexpr (FUSED) {  // the tokens' positions and slots, read during the weight stream
        if (tid < kBgTile * TT) {
            const int t = min(t0 + tid, a.m - 1);
            s_pos[tid] = a.d_positions[t];
            s_slot[tid] = a.d_slots[t];
        }
    }

    float4v_t acc[TT], f[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[tt][r] = f[tt][r] = 0.0f;
    for (int c0 = 0; c0 < chunks; c0 += DEPTH) {
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) {
            const int c = c0 + i;
            if (c < chunks) {
                const float sc = h2f(sq[i]);
                half8_t wb[XV];
                if constexpr (KC == 64) {
                    wb[0] = e4m3x8(wq[i].v.x, wq[i].v.y);
                    wb[XV - 1] = e4m3x8(wq[i].v.z, wq[i].v.w);
                } else {
                    wb[0] = e4m3x8(wq[i].v.x, wq[i].v.y);
                }
                half8_t xa[TT][XV];
                if constexpr (KC == 64) {
                    // Through the LDS stage: MFMA v takes piece 2 sub + v of token j.
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
                        for (int v = 0; v < 2; ++v) {
                            // (a value store: storing the array element directly became a
                            // copy out of private memory and kept xq in scratch)
                            const uint4 val = xq[i][tt][v];
                            s_x[part][tt][v][lane] = make_uint4(val.x, val.y, val.z, val.w);
                        }
                    // The stage writes and reads index one LDS array at run time, so the
                    // compiler keeps their order; the wait orders them in the LDS queue.
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
                        for (int v = 0; v < 2; ++v) {
                            const int q = 2 * sub + v;
                            const int pos = 8 * (j & 7) + (q ^ ((j >> 1) & 7));
                            xa[tt][v] = __builtin_bit_cast(half8_t, s_x[part][tt][j >> 3][pos]);
                        }
                } else {
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt)
                        xa[tt][0] = __builtin_bit_cast(half8_t, xq[i][tt][0]);
                }
                if (c + DEPTH < chunks) issue(i, c + DEPTH);  // refill the slot DEPTH chunks ahead
#pragma unroll
                for (int v = 0; v < XV; ++v)
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt)
                        f[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[tt][v], wb[v], f[tt], 0, 0, 0);
                if ((c + 1) % per_group == 0) {  // group done: scale into the accumulator
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            acc[tt][r] = fmaf(sc, f[tt][r], acc[tt][r]);
                            f[tt][r] = 0.0f;
                        }
                }
            }
        }
    }

    // Sum the parts in a fixed order (part 0 + 1 + ... + 7) through LDS.
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_red[part][tt * 4 + r][lane] = acc[tt][r];
    __syncthreads();
    if (part != 0) return;
#pragma unroll
    for (int q = 0; q < TT * 4; ++q) {
        float v = s_red[0][q][lane];
#pragma unroll
        for (int p = 1; p < kBgParts; ++p) v += s_red[p][q][lane];
        acc[q >> 2][q & 3] = v;
    }

    // Register r of token tile tt, lane l: token t0 + 16 tt + 4 (l/16) + r, weight row `row`.
    if constexpr (!FUSED) {
        if (row >= a.n) return;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = t0 + kBgTile * tt + 4 * sub + r;
                if (t < a.m) a.y[size_t(t) * a.y_stride + row] = f2h(acc[tt][r]);
            }
    } else {
        const int hd = a.head_dim, half = hd / 2;
        const int head = blk >> 3;
        const bool lo = j < 8;               // this lane holds dim d; lane ^ 8 holds d + 64
        const int d = (blk & 7) * 8 + (j & 7);  // pair index, 0 .. 63
        const int dim = lo ? d : d + half;      // the element this lane writes
        const int kind = head < a.n_q_heads ? 0 : (head < a.n_q_heads + a.n_kv_heads ? 1 : 2);
        const int kh = head - a.n_q_heads - (kind == 2 ? a.n_kv_heads : 0);
        const int kv_dim = a.n_kv_heads * hd;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint16_t mine = f2h(acc[tt][r]);
                const uint16_t other = uint16_t(__shfl_xor(int(mine), 8));
                const int t = t0 + kBgTile * tt + 4 * sub + r;
                if (t >= a.m) continue;
                uint16_t* yrow = a.y + size_t(t) * a.y_stride + size_t(head) * hd;
                const int pos = s_pos[t - t0];
                const int64_t slot = s_slot[t - t0];
                if (pos < 0 || pos >= a.max_pos || slot < 0 || slot >= a.max_rows) {
                    // nothing is rotated or appended for an out-of-range token
                    yrow[dim] = mine;
                    if (a.d_status && j == 0) *a.d_status = AF_ERR_OUT_OF_RANGE;
                    continue;
                }
                const uint16_t y0 = lo ? mine : other, y1 = lo ? other : mine;
                uint16_t o0 = y0, o1 = y1;
                if (kind < 2)
                    rope_rotate(y0, y1, a.cos_t[size_t(pos) * half + d],
                                a.sin_t[size_t(pos) * half + d], o0, o1);
                const uint16_t out = lo ? o0 : o1;
                yrow[dim] = out;
                if (kind > 0) {
                    const size_t e = size_t(slot) * kv_dim + size_t(kh) * hd + dim;
                    uint8_t* base = kind == 1 ? a.k_dst : a.v_dst;
                    if constexpr (FP8) {
                        const float sc = (kind == 1 ? a.k_scales : a.v_scales)[kh];
                        base[e] = uint8_t(quantize_fp8(out, sc));
                    } else {
                        reinterpret_cast<uint16_t*>(base)[e] = out;
                    }
                }
            }
    }
}

template <bool FUSED, bool FP8>
void launch_batched(const BatchedArgs& a, int row_blocks, hipStream_t s) {
    const bool two = a.m > kBgTile;
    const int per = kBgTile * (two ? 2 : 1);
    const dim3 grid(row_blocks, (a.m + per - 1) / per), block(kBgThreads);
    const bool k64 = a.group_size % 64 == 0;
    if (two) {
        if (k64) hipLaunchKernelGGL((w8a16_batched_kernel<FUSED, FP8, 2, 64>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((w8a16_batched_kernel<FUSED, FP8, 2, 32>), grid, block, 0, s, a);
    } else {
        if (k64) hipLaunchKernelGGL((w8a16_batched_kernel<FUSED, FP8, 1, 64>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((w8a16_batched_kernel<FUSED, FP8, 1, 32>), grid, block, 0, s, a);
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
    // One token: the single-token GEMV streams the weights faster than one
    // 16-token MFMA tile that is 15/16 padding.
    if (m == 1) return af_w8a16_gemv(x, weight, scales, y, n, k, group_size, stream);
    BatchedArgs a{};
    fill_common(a, x, x_stride, m, weight, scales, n, k, group_size);
    a.y = static_cast<uint16_t*>(y);
    a.y_stride = y_stride;
    launch_batched<false, false>(a, (n + kBgRows - 1) / kBgRows, static_cast<hipStream_t>(stream));
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
    if (pool->flags & ~AF_KV_POOL_SHARED_BLOCKS) return AF_ERR_INVALID_ARG;
    const bool fp8 = pool->dtype == AF_KV_FP8_E4M3;
    if (!fp8 && pool->dtype != AF_KV_FP16) return AF_ERR_UNSUPPORTED;
    if (fp8 && !pool->scales) return AF_ERR_INVALID_ARG;
    if (pool->n_kv_heads <= 0) return AF_ERR_INVALID_ARG;
    const int hd = pool->head_dim;
    if (hd != 128) return AF_ERR_UNSUPPORTED;  // a workgroup's columns are d and d + 64
    const int n = (n_q_heads + 2 * pool->n_kv_heads) * hd;
    if (int st = check_batched(x, x_stride, m, w_qkv, scales, n, k, group_size)) return st;
    if (m == 0) return AF_OK;
    const size_t esz = fp8 ? 1 : 2;
    const int kv_dim = pool->n_kv_heads * hd;
    const size_t slab = size_t(pool->total_blocks) * pool->block_size * kv_dim * esz;
    uint8_t* base = static_cast<uint8_t*>(pool->base);
    if (m == 1) {  // one token: the GEMV form, as af_w8a16_gemm_batched at m = 1
        QkvSingleArgs q{};
        q.w = w_qkv;
        q.x = static_cast<const uint16_t*>(x);
        q.scales = static_cast<const uint16_t*>(scales);
        q.k = k;
        q.group_size = group_size;
        q.qkv = static_cast<uint16_t*>(qkv_out);
        q.k_dst = base + size_t(2 * layer) * slab;
        q.v_dst = base + size_t(2 * layer + 1) * slab;
        q.cos_t = cos_table;
        q.sin_t = sin_table;
        q.d_pos = d_positions;
        q.max_pos = max_pos;
        q.d_slot = d_slots;
        q.max_rows = int64_t(pool->total_blocks) * pool->block_size;
        if (fp8) {
            q.k_scales = pool->scales + size_t(layer) * 2 * pool->n_kv_heads;
            q.v_scales = q.k_scales + pool->n_kv_heads;
        }
        q.n_q_heads = n_q_heads;
        q.n_kv_heads = pool->n_kv_heads;
        q.head_dim = hd;
        q.d_status = d_status;
        launch_qkv_single(q, fp8 ? kQkvPagedFp8 : kQkvPagedFp16, static_cast<hipStream_t>(stream));
        AF_TRY_LAUNCH();
        return AF_OK;
    }
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
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (fp8)
        launch_batched<true, true>(a, n / kBgRows, s);  // eight workgroups per head
    else
        launch_batched<true, false>(a, n / kBgRows, s);
    AF_TRY_LAUNCH();
    return AF_OK;
}
