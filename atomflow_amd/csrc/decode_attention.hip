// decode_attention.hip — GQA decode attention (M = 1 query token per sequence)
// over the contiguous cache and the paged pool, fp16 or FP8-E4M3 KV, gfx950.
//
// Computes, for every query head h of every sequence b (the reference's
// gqa_cached_attention_kernel, src/kernel/tiled_attention.cu:196-269):
//     out[h] = softmax_t(q_h . K[t, kv(h)] / sqrt(hd)) . V[:, kv(h)],  t < L_b
// with kv(h) = h / GROUP (tiled_attention.cu:208).
//
// Design (bandwidth-bound: 3 flop per KV byte for fp16, no MFMA):
//  * Split-K over the sequence ("flash decoding"): workgroup = (sequence,
//    KV head, split). The GROUP query heads of a KV head share every K/V byte
//    (the reference reads each KV head once per query head).
//  * Linear workgroup id = ((b * splits) + split) * n_kv_heads + kv_head, so
//    with 8 KV heads every split of KV head h lands on XCD h (workgroups are
//    dealt round-robin over the 8 XCDs): the partials a head's combine reads
//    were written through the same L2.
//  * A token row of one head is 8 lanes x 16 B (fp16: two loads per lane, fp8:
//    one): every load instruction reads whole 128-B lines. QK partial dots are
//    summed across the 8 lanes with three DPP adds; the softmax max is made
//    wave-uniform per chunk so the accumulator rescale is a uniform branch.
//  * fp32 online softmax (exp2 with log2(e) folded into the score scale), fp32
//    accumulation via v_fma_mix (fp16 V) or v_cvt_pk_f32_fp8 (FP8 V).
//  * The last workgroup of a (sequence, KV head) to finish merges the splits'
//    (m, l, o[]) partials and writes fp16 output; it also re-zeroes the arrival
//    counter, so the kernel is one launch and replays inside a hipGraph.
//  * Paged: the split's block-table entries are staged in LDS once; rows are
//    addressed block * block_size + (t mod block_size) within the layer slab.
#include <cmath>
#include <mutex>
#include <vector>

#include "af_common.h"

namespace af {
namespace {

typedef _Float16 f16;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;              // waves per workgroup
constexpr int kThreads = kWaves * 64;  // 256
constexpr int kLanesPerRow = 8;        // lanes that share one token row of one head
constexpr int kRowsPerStep = 64 / kLanesPerRow;  // 8 tokens per wave load step
constexpr int kMaxTableLds = 1024;     // block-table entries staged per split

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Sum over the 8 lanes of a token group; every lane receives the same bits.
__device__ __forceinline__ float group8_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror: pairs the two quads of each 8-lane half
    return v;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Max over the wave of a value that is uniform within each 8-lane group.
__device__ __forceinline__ float wave_max_of_groups(float v) {
    v = fmaxf(v, dpp<0x128>(v));  // row_ror:8 joins the two groups of a 16-lane row
    const float a = readlane_f(v, 0), b = readlane_f(v, 16);
    const float c = readlane_f(v, 32), d = readlane_f(v, 48);
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int ceil_div_d(int a, int b) { return (a + b - 1) / b; }

struct AttnArgs {
    const uint16_t* q;
    int64_t q_stride;  // elements between sequences
    const uint8_t* k;  // contiguous cache base, or the layer's K slab
    const uint8_t* v;
    int64_t row_bytes;  // bytes between consecutive token rows (kv_dim * elem)
    const int32_t* tables;
    int32_t max_blocks;
    int32_t block_shift;
    int64_t total_blocks;
    const int32_t* seq_lens;  // [batch] or NULL -> seq_len_host
    int32_t seq_len_host;
    int32_t max_seq_len;
    uint16_t* out;
    int64_t out_stride;
    int32_t n_kv_heads;
    int32_t num_splits;
    int32_t min_span;
    float qk_scale;       // log2(e) / sqrt(head_dim)
    const float* scales;  // FP8: [2][n_kv_heads] (K, V) of this layer
    float* part_o;
    float* part_ml;
    uint32_t* counters;
};

template <int HD, bool FP8>
struct Layout {
    static constexpr int kElem = FP8 ? 1 : 2;
    static constexpr int kRowBytes = HD * kElem;                   // one head, one token
    static constexpr int kLoads = kRowBytes / (kLanesPerRow * 16);  // 16-B loads per lane per row
    static constexpr int kElemsPerLoad = 16 / kElem;
    static constexpr int kEpl = kLoads * kElemsPerLoad;  // elements per lane per row
    static_assert(kLoads >= 1, "head row must span 8 lanes x 16 B");
    // head-dim index of element u of load i for lane j
    __device__ static int dim(int i, int j, int u) { return (i * 128 + j * 16) / kElem + u; }
};

template <int HD, int GROUP, bool FP8, bool PAGED>
__global__ __launch_bounds__(kThreads) void decode_attn_kernel(const AttnArgs a) {
    using LY = Layout<HD, FP8>;
    constexpr int LOADS = LY::kLoads;
    constexpr int EPL = LY::kEpl;
    constexpr int R = 2;                           // token rows per lane per chunk
    constexpr int CHUNK = R * kRowsPerStep;        // tokens per wave chunk (16)

    __shared__ float s_o[kWaves][GROUP][HD];
    __shared__ float s_m[kWaves][GROUP];
    __shared__ float s_l[kWaves][GROUP];
    __shared__ int32_t s_tab[PAGED ? kMaxTableLds : 1];
    __shared__ float s_w[GROUP][kMaxSplits];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 3, j = lane & 7;
    int id = blockIdx.x;
    const int h = id % a.n_kv_heads;
    id /= a.n_kv_heads;
    const int split = id % a.num_splits;
    const int b = id / a.num_splits;
    const int nq = a.n_kv_heads * GROUP;

    int L = a.seq_lens ? a.seq_lens[b] : a.seq_len_host;
    L = min(L, a.max_seq_len);
    uint16_t* out_b = a.out + size_t(b) * a.out_stride + size_t(h) * GROUP * HD;
    if (L <= 0) {  // empty sequence: defined as a zero output
        if (split == 0)
            for (int o = tid; o < GROUP * HD; o += kThreads) out_b[o] = 0;
        return;
    }
    int span = max(ceil_div_d(L, a.num_splits), a.min_span);
    span = (span + CHUNK - 1) / CHUNK * CHUNK;
    const int n_active = (L + span - 1) / span;
    if (split >= n_active) return;
    const int t_begin = split * span;
    const int t_end = min(L, t_begin + span);

    // ---- stage this split's block-table entries (paged) --------------------
    int tab_base = 0;
    if constexpr (PAGED) {
        const int first = t_begin >> a.block_shift;
        const int last = (t_end - 1) >> a.block_shift;
        tab_base = first;
        const int32_t* trow = a.tables + size_t(b) * a.max_blocks;
        for (int e = tid; e <= last - first; e += kThreads) {
            int blk = trow[first + e];
            blk = min(max(blk, 0), int(a.total_blocks - 1));  // never address outside the pool
            s_tab[e] = blk;
        }
        __syncthreads();
    }

    // ---- query fragment: the lane's EPL dims of each of the GROUP heads ----
    half2_t qv[GROUP][EPL / 2];
    {
        const uint16_t* qb = a.q + size_t(b) * a.q_stride + size_t(h) * GROUP * HD;
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh)
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                const uint16_t* src = qb + gh * HD + LY::dim(i, j, 0);
#pragma unroll
                for (int w = 0; w < LY::kElemsPerLoad / 8; ++w) {
                    const uint4 raw = *reinterpret_cast<const uint4*>(src + w * 8);
                    const int p0 = i * (LY::kElemsPerLoad / 2) + w * 4;
                    qv[gh][p0 + 0] = __builtin_bit_cast(half2_t, raw.x);
                    qv[gh][p0 + 1] = __builtin_bit_cast(half2_t, raw.y);
                    qv[gh][p0 + 2] = __builtin_bit_cast(half2_t, raw.z);
                    qv[gh][p0 + 3] = __builtin_bit_cast(half2_t, raw.w);
                }
            }
    }

    float qk_scale = a.qk_scale;
    float v_scale = 1.0f;
    if constexpr (FP8) {
        qk_scale *= a.scales[h];
        v_scale = a.scales[a.n_kv_heads + h];
    }

    float m_run[GROUP], l_run[GROUP], acc[GROUP][EPL];
#pragma unroll
    for (int gh = 0; gh < GROUP; ++gh) {
        m_run[gh] = -INFINITY;
        l_run[gh] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[gh][e] = 0.f;
    }

    const int n_chunks = (t_end - t_begin + CHUNK - 1) / CHUNK;
    const uint8_t* kbase = a.k + size_t(h) * LY::kRowBytes + j * 16;
    const uint8_t* vbase = a.v + size_t(h) * LY::kRowBytes + j * 16;

    struct Chunk {
        uint4 k[R][LOADS];
        uint4 v[R][LOADS];
    };

    auto row_offset = [&](int t) -> int64_t {
        const int tc = min(t, L - 1);  // rows past L are read from row L-1 and masked
        if constexpr (PAGED) {
            const int mask = (1 << a.block_shift) - 1;
            const int64_t blk = s_tab[(tc >> a.block_shift) - tab_base];
            return ((blk << a.block_shift) | (tc & mask)) * a.row_bytes;
        } else {
            return int64_t(tc) * a.row_bytes;
        }
    };

    auto load_chunk = [&](Chunk& c, int chunk) {
        const int t0 = t_begin + chunk * CHUNK + g;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t off = row_offset(t0 + r * kRowsPerStep);
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                c.k[r][i] = *reinterpret_cast<const uint4*>(kbase + off + i * 128);
                c.v[r][i] = *reinterpret_cast<const uint4*>(vbase + off + i * 128);
            }
        }
    };

    auto process_chunk = [&](const Chunk& c, int chunk) {
        const int t0 = t_begin + chunk * CHUNK + g;
        float s[R][GROUP];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int gh = 0; gh < GROUP; ++gh) s[r][gh] = 0.f;
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                const uint32_t w4[4] = {c.k[r][i].x, c.k[r][i].y, c.k[r][i].z, c.k[r][i].w};
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    if constexpr (FP8) {
                        const half2_t k01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(w4[w]), 1.0f, false);
                        const half2_t k23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(w4[w]), 1.0f, true);
                        const int p = i * 8 + w * 2;
#pragma unroll
                        for (int gh = 0; gh < GROUP; ++gh) {
                            s[r][gh] = __builtin_amdgcn_fdot2(k01, qv[gh][p], s[r][gh], false);
                            s[r][gh] = __builtin_amdgcn_fdot2(k23, qv[gh][p + 1], s[r][gh], false);
                        }
                    } else {
                        const half2_t kk = __builtin_bit_cast(half2_t, w4[w]);
                        const int p = i * 4 + w;
#pragma unroll
                        for (int gh = 0; gh < GROUP; ++gh)
                            s[r][gh] = __builtin_amdgcn_fdot2(kk, qv[gh][p], s[r][gh], false);
                    }
                }
            }
        }
        float cmax[GROUP];
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh) cmax[gh] = -INFINITY;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool valid = (t0 + r * kRowsPerStep) < t_end;
#pragma unroll
            for (int gh = 0; gh < GROUP; ++gh) {
                const float x = group8_sum(s[r][gh]) * qk_scale;
                s[r][gh] = valid ? x : -INFINITY;
                cmax[gh] = fmaxf(cmax[gh], s[r][gh]);
            }
        }
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh) {
            const float m_new = fmaxf(m_run[gh], wave_max_of_groups(cmax[gh]));
            if (m_new > m_run[gh]) {  // wave-uniform
                const float alpha = fast_exp2(m_run[gh] - m_new);
                l_run[gh] *= alpha;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[gh][e] *= alpha;
                m_run[gh] = m_new;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float p[GROUP];
#pragma unroll
            for (int gh = 0; gh < GROUP; ++gh) {
                p[gh] = fast_exp2(s[r][gh] - m_run[gh]);
                l_run[gh] += p[gh];
            }
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                const uint32_t w4[4] = {c.v[r][i].x, c.v[r][i].y, c.v[r][i].z, c.v[r][i].w};
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    if constexpr (FP8) {
                        const float2_t v01 = __builtin_amdgcn_cvt_pk_f32_fp8(int(w4[w]), false);
                        const float2_t v23 = __builtin_amdgcn_cvt_pk_f32_fp8(int(w4[w]), true);
                        const int e = i * 16 + w * 4;
#pragma unroll
                        for (int gh = 0; gh < GROUP; ++gh) {
                            acc[gh][e + 0] = fmaf(p[gh], v01[0], acc[gh][e + 0]);
                            acc[gh][e + 1] = fmaf(p[gh], v01[1], acc[gh][e + 1]);
                            acc[gh][e + 2] = fmaf(p[gh], v23[0], acc[gh][e + 2]);
                            acc[gh][e + 3] = fmaf(p[gh], v23[1], acc[gh][e + 3]);
                        }
                    } else {
                        const half2_t vv = __builtin_bit_cast(half2_t, w4[w]);
                        const int e = i * 8 + w * 2;
#pragma unroll
                        for (int gh = 0; gh < GROUP; ++gh) {
                            acc[gh][e + 0] = fmaf(p[gh], float(vv[0]), acc[gh][e + 0]);
                            acc[gh][e + 1] = fmaf(p[gh], float(vv[1]), acc[gh][e + 1]);
                        }
                    }
                }
            }
        }
    };

    // ---- main loop: wave w takes chunks w, w+4, ...; one chunk prefetched ---
    {
        Chunk ca, cb;
        int c = wave;
        if (c < n_chunks) load_chunk(ca, c);
        while (c < n_chunks) {
            if (c + kWaves < n_chunks) load_chunk(cb, c + kWaves);
            process_chunk(ca, c);
            c += kWaves;
            if (c >= n_chunks) break;
            if (c + kWaves < n_chunks) load_chunk(ca, c + kWaves);
            process_chunk(cb, c);
            c += kWaves;
        }
    }

    // ---- merge the wave's 8 token groups (m is wave-uniform: plain sums) ----
#pragma unroll
    for (int gh = 0; gh < GROUP; ++gh) {
        float l = l_run[gh];
        l += dpp<0x128>(l);
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        l_run[gh] = l;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float x = acc[gh][e];
            x += dpp<0x128>(x);
            x += __shfl_xor(x, 16);
            x += __shfl_xor(x, 32);
            acc[gh][e] = x;
        }
    }
    if (lane < kLanesPerRow) {
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh) {
#pragma unroll
            for (int i = 0; i < LOADS; ++i)
#pragma unroll
                for (int u = 0; u < LY::kElemsPerLoad; ++u)
                    s_o[wave][gh][LY::dim(i, j, u)] = acc[gh][i * LY::kElemsPerLoad + u];
            if (lane == 0) {
                s_m[wave][gh] = m_run[gh];
                s_l[wave][gh] = l_run[gh];
            }
        }
    }
    __syncthreads();

    // ---- merge the 4 waves; write the output or this split's partial -------
    for (int o = tid; o < GROUP * HD; o += kThreads) {
        const int gh = o / HD, d = o % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][gh]);
        float lsum = 0.f, osum = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float f = fast_exp2(s_m[w][gh] - M);  // 0 for a wave that saw no token
            lsum += f * s_l[w][gh];
            osum += f * s_o[w][gh][d];
        }
        if (n_active == 1) {
            out_b[o] = __builtin_bit_cast(uint16_t, f16(osum * v_scale / lsum));
        } else {
            const size_t qh = size_t(b) * nq + size_t(h) * GROUP + gh;
            const size_t slot = qh * a.num_splits + split;
            a.part_o[slot * HD + d] = osum * v_scale;
            if (d == 0) {
                a.part_ml[slot * 2 + 0] = M;
                a.part_ml[slot * 2 + 1] = lsum;
            }
        }
    }
    if (n_active == 1) return;

    // ---- arrival: the last split of (b, h) to finish combines --------------
    __threadfence();  // each wave publishes its partial stores device-wide
    __syncthreads();
    if (tid == 0) {
        uint32_t* ctr = a.counters + size_t(b) * a.n_kv_heads + h;
        const uint32_t prev = atomicAdd(ctr, 1u);
        const int last = prev == uint32_t(n_active - 1);
        if (last) *ctr = 0u;  // every other split has arrived: safe to re-arm
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();  // acquire the other splits' partials

    for (int gh = wave; gh < GROUP; gh += kWaves) {
        const size_t qh = size_t(b) * nq + size_t(h) * GROUP + gh;
        const float* ml = a.part_ml + qh * a.num_splits * 2;
        float mx = -INFINITY;
        for (int s = lane; s < n_active; s += 64) mx = fmaxf(mx, ml[s * 2]);
        mx = wave_max(mx);
        float ls = 0.f;
        for (int s = lane; s < n_active; s += 64) {
            const float w = fast_exp2(ml[s * 2] - mx);
            s_w[gh][s] = w;
            ls += w * ml[s * 2 + 1];
        }
        ls = wave_sum(ls);
        const float inv = 1.0f / ls;
        for (int s = lane; s < n_active; s += 64) s_w[gh][s] *= inv;
    }
    __syncthreads();
    for (int o = tid; o < GROUP * HD; o += kThreads) {
        const int gh = o / HD, d = o % HD;
        const size_t qh = size_t(b) * nq + size_t(h) * GROUP + gh;
        const float* po = a.part_o + qh * a.num_splits * HD + d;
        float x = 0.f;
        for (int s = 0; s < n_active; ++s) x = fmaf(s_w[gh][s], po[size_t(s) * HD], x);
        out_b[o] = __builtin_bit_cast(uint16_t, f16(x));
    }
}

}  // namespace
}  // namespace af

// ============================================================================
// Host side: dispatch, split heuristics, workspaces, C ABI.
// ============================================================================
namespace af {
namespace {

template <int HD, int GROUP, bool FP8, bool PAGED>
hipError_t launch_attn(const AttnArgs& a, int grid, hipStream_t s) {
    hipLaunchKernelGGL((decode_attn_kernel<HD, GROUP, FP8, PAGED>), dim3(grid), dim3(kThreads), 0,
                       s, a);
    return hipGetLastError();
}

template <int HD, bool FP8, bool PAGED>
int dispatch_group(const AttnArgs& a, int group, int grid, hipStream_t s) {
    switch (group) {
        case 1: return int(launch_attn<HD, 1, FP8, PAGED>(a, grid, s));
        case 2: return int(launch_attn<HD, 2, FP8, PAGED>(a, grid, s));
        case 3: return int(launch_attn<HD, 3, FP8, PAGED>(a, grid, s));
        case 4: return int(launch_attn<HD, 4, FP8, PAGED>(a, grid, s));
        case 8: return int(launch_attn<HD, 8, FP8, PAGED>(a, grid, s));
        default: return AF_ERR_UNSUPPORTED;
    }
}

int dispatch(const AttnArgs& a, int head_dim, int group, bool fp8, bool paged, int grid,
             hipStream_t s) {
    if (fp8) {
        if (!paged || head_dim != 128) return AF_ERR_UNSUPPORTED;
        return dispatch_group<128, true, true>(a, group, grid, s);
    }
    if (head_dim == 128)
        return paged ? dispatch_group<128, false, true>(a, group, grid, s)
                     : dispatch_group<128, false, false>(a, group, grid, s);
    if (head_dim == 64)
        return paged ? dispatch_group<64, false, true>(a, group, grid, s)
                     : dispatch_group<64, false, false>(a, group, grid, s);
    return AF_ERR_UNSUPPORTED;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

float qk_scale_for(int head_dim) { return float(1.4426950408889634 / std::sqrt(double(head_dim))); }

// Library-owned workspace of af_cached_attention (one per device).
struct OwnedWorkspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::vector<OwnedWorkspace> g_ws;

int owned_workspace(int batch, int n_q_heads, int head_dim, hipStream_t stream, void** ptr,
                    size_t* bytes) {
    int dev = 0;
    AF_TRY_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if (int(g_ws.size()) <= dev) g_ws.resize(dev + 1);
    OwnedWorkspace& w = g_ws[dev];
    const size_t need = attn_workspace_bytes(batch, n_q_heads, head_dim, kMaxSplits);
    if (w.bytes < need) {
        if (stream) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            AF_TRY_HIP(hipStreamIsCapturing(stream, &cs));
            if (cs != hipStreamCaptureStatusNone) return AF_ERR_WORKSPACE;  // reserve first
        }
        if (w.ptr) {
            AF_TRY_HIP(hipDeviceSynchronize());
            AF_TRY_HIP(hipFree(w.ptr));
            w.ptr = nullptr;
            w.bytes = 0;
        }
        void* p = nullptr;
        AF_TRY_HIP(hipMalloc(&p, need));
        int st = fill_u32(p, 0u, kCounterBytes / 4, stream);
        if (st) {
            (void)hipFree(p);
            return st;
        }
        w.ptr = p;
        w.bytes = need;
    }
    *ptr = w.ptr;
    *bytes = w.bytes;
    return AF_OK;
}

}  // namespace

int device_compute_units() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (int(cache.size()) <= dev) cache.resize(dev + 1, 0);
    if (!cache[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cache[dev] = cus;
    }
    return cache[dev];
}

int default_splits(int max_seq_len, int batch, int n_kv_heads) {
    if (max_seq_len <= 0) return 1;
    const int pairs = std::max(1, batch * n_kv_heads);
    int splits = ceil_div(2 * device_compute_units(), pairs);
    splits = std::max(splits, ceil_div(max_seq_len, 1024));  // long sequences: bounded spans
    splits = std::min(splits, std::max(1, ceil_div(max_seq_len, kMinSpan)));
    return std::min(std::max(splits, 1), kMaxSplits);
}

// Smallest split count whose span fits the LDS-staged block table.
static int min_splits_for_table(int max_seq_len, int block_size) {
    const int max_span = (kMaxTableLds - 2) * block_size - 16;
    return ceil_div(max_seq_len, max_span);
}

}  // namespace af

using namespace af;

extern "C" size_t af_attention_workspace_size(int batch, int n_q_heads, int n_kv_heads,
                                              int head_dim, int num_splits) {
    if (batch <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0) return 0;
    if (num_splits <= 0 || num_splits > kMaxSplits) num_splits = kMaxSplits;
    return attn_workspace_bytes(batch, n_q_heads, head_dim, num_splits);
}

extern "C" int af_attention_workspace_init(void* workspace, size_t workspace_bytes,
                                           af_stream_t stream) {
    if (!workspace || workspace_bytes < kCounterBytes) return AF_ERR_WORKSPACE;
    return fill_u32(workspace, 0u, kCounterBytes / 4, static_cast<hipStream_t>(stream));
}

extern "C" int af_attention_default_splits(int max_seq_len, int batch, int n_kv_heads) {
    return default_splits(max_seq_len, batch, n_kv_heads);
}

static int check_heads(int head_dim, int n_q_heads, int n_kv_heads) {
    if (head_dim <= 0 || n_q_heads <= 0 || n_kv_heads <= 0) return AF_ERR_INVALID_ARG;
    if (n_q_heads % n_kv_heads) return AF_ERR_UNSUPPORTED;
    return AF_OK;
}

extern "C" int af_cached_attention_ex(const void* q, const void* k_cache, const void* v_cache,
                                      void* out, int seq_len, const int32_t* d_seq_len,
                                      int max_seq_len, int head_dim, int n_q_heads, int n_kv_heads,
                                      int num_splits, void* workspace, size_t workspace_bytes,
                                      af_stream_t stream) {
    if (!q || !k_cache || !v_cache || !out || max_seq_len <= 0) return AF_ERR_INVALID_ARG;
    if (int st = check_heads(head_dim, n_q_heads, n_kv_heads)) return st;
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache)) return AF_ERR_INVALID_ARG;
    if (!d_seq_len && (seq_len < 0 || seq_len > max_seq_len)) return AF_ERR_OUT_OF_RANGE;
    if (num_splits <= 0) num_splits = default_splits(max_seq_len, 1, n_kv_heads);
    if (num_splits > kMaxSplits) return AF_ERR_INVALID_ARG;
    if (n_kv_heads > kMaxCounters) return AF_ERR_UNSUPPORTED;
    if (!workspace || workspace_bytes < attn_workspace_bytes(1, n_q_heads, head_dim, num_splits))
        return AF_ERR_WORKSPACE;
    const AttnWorkspace w = attn_workspace_carve(workspace, 1, n_q_heads, num_splits);
    AttnArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.q_stride = int64_t(n_q_heads) * head_dim;
    a.k = static_cast<const uint8_t*>(k_cache);
    a.v = static_cast<const uint8_t*>(v_cache);
    a.row_bytes = int64_t(n_kv_heads) * head_dim * 2;
    a.seq_lens = d_seq_len;
    a.seq_len_host = seq_len;
    a.max_seq_len = max_seq_len;
    a.out = static_cast<uint16_t*>(out);
    a.out_stride = int64_t(n_q_heads) * head_dim;
    a.n_kv_heads = n_kv_heads;
    a.num_splits = num_splits;
    a.min_span = kMinSpan;
    a.qk_scale = qk_scale_for(head_dim);
    a.part_o = w.part_o;
    a.part_ml = w.part_ml;
    a.counters = w.counters;
    const int grid = num_splits * n_kv_heads;
    return dispatch(a, head_dim, n_q_heads / n_kv_heads, false, false, grid,
                    static_cast<hipStream_t>(stream));
}

extern "C" int af_attention_reserve(int batch, int n_q_heads, int n_kv_heads, int head_dim) {
    if (batch <= 0) return AF_ERR_INVALID_ARG;
    if (int st = check_heads(head_dim, n_q_heads, n_kv_heads)) return st;
    void* p = nullptr;
    size_t bytes = 0;
    int st = owned_workspace(batch, n_q_heads, head_dim, nullptr, &p, &bytes);
    if (st) return st;
    return int(hipDeviceSynchronize());
}

extern "C" int af_cached_attention(const void* q, const void* k_cache, const void* v_cache,
                                   void* out, int seq_len, int head_dim, int n_q_heads,
                                   int n_kv_heads, af_stream_t stream) {
    if (seq_len <= 0) return AF_ERR_INVALID_ARG;  // the reference attends over pos+1 >= 1 tokens
    if (int st = check_heads(head_dim, n_q_heads, n_kv_heads)) return st;
    void* ws = nullptr;
    size_t bytes = 0;
    int st = owned_workspace(1, n_q_heads, head_dim, static_cast<hipStream_t>(stream), &ws, &bytes);
    if (st) return st;
    return af_cached_attention_ex(q, k_cache, v_cache, out, seq_len, nullptr, seq_len, head_dim,
                                  n_q_heads, n_kv_heads, default_splits(seq_len, 1, n_kv_heads), ws,
                                  bytes, stream);
}

extern "C" int af_paged_attention(const void* q, int q_stride, const af_kv_pool* pool, int layer,
                                  const int32_t* d_block_tables, int max_blocks_per_seq,
                                  const int32_t* d_seq_lens, int batch, int max_seq_len, void* out,
                                  int out_stride, int n_q_heads, int num_splits, void* workspace,
                                  size_t workspace_bytes, af_stream_t stream) {
    if (!q || !pool || !pool->base || !d_block_tables || !d_seq_lens || !out || batch < 0 ||
        max_seq_len < 0 || max_blocks_per_seq <= 0)
        return AF_ERR_INVALID_ARG;
    if (layer < 0 || layer >= pool->n_layers) return AF_ERR_INVALID_ARG;
    const int hd = pool->head_dim, nkv = pool->n_kv_heads;
    if (int st = check_heads(hd, n_q_heads, nkv)) return st;
    const int bs = pool->block_size;
    if (bs < 8 || (bs & (bs - 1))) return AF_ERR_UNSUPPORTED;
    const bool fp8 = pool->dtype == AF_KV_FP8_E4M3;
    if (!fp8 && pool->dtype != AF_KV_FP16) return AF_ERR_UNSUPPORTED;
    if (fp8 && !pool->scales) return AF_ERR_INVALID_ARG;
    if (q_stride < n_q_heads * hd || out_stride < n_q_heads * hd) return AF_ERR_INVALID_ARG;
    if (!aligned16(q) || !aligned16(pool->base) || (q_stride % 8)) return AF_ERR_INVALID_ARG;
    if (int64_t(max_blocks_per_seq) * bs < max_seq_len) return AF_ERR_OUT_OF_RANGE;
    if (batch == 0) return AF_OK;
    if (int64_t(batch) * nkv > kMaxCounters) return AF_ERR_UNSUPPORTED;
    const int min_sp = min_splits_for_table(std::max(max_seq_len, 1), bs);
    if (num_splits <= 0)
        num_splits = std::max(default_splits(max_seq_len, batch, nkv), min_sp);
    else if (num_splits < min_sp)
        return AF_ERR_INVALID_ARG;
    if (num_splits > kMaxSplits) return AF_ERR_OUT_OF_RANGE;
    if (!workspace || workspace_bytes < attn_workspace_bytes(batch, n_q_heads, hd, num_splits))
        return AF_ERR_WORKSPACE;
    const AttnWorkspace w = attn_workspace_carve(workspace, batch, n_q_heads, num_splits);
    const size_t esz = fp8 ? 1 : 2;
    const size_t slab = size_t(pool->total_blocks) * bs * nkv * hd * esz;
    const uint8_t* base = static_cast<const uint8_t*>(pool->base);
    AttnArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.q_stride = q_stride;
    a.k = base + size_t(2 * layer) * slab;
    a.v = base + size_t(2 * layer + 1) * slab;
    a.row_bytes = int64_t(nkv) * hd * esz;
    a.tables = d_block_tables;
    a.max_blocks = max_blocks_per_seq;
    a.block_shift = __builtin_ctz(unsigned(bs));
    a.total_blocks = pool->total_blocks;
    a.seq_lens = d_seq_lens;
    a.seq_len_host = 0;
    a.max_seq_len = max_seq_len;
    a.out = static_cast<uint16_t*>(out);
    a.out_stride = out_stride;
    a.n_kv_heads = nkv;
    a.num_splits = num_splits;
    a.min_span = kMinSpan;
    a.qk_scale = qk_scale_for(hd);
    a.scales = fp8 ? pool->scales + size_t(layer) * 2 * nkv : nullptr;
    a.part_o = w.part_o;
    a.part_ml = w.part_ml;
    a.counters = w.counters;
    const int64_t grid = int64_t(batch) * num_splits * nkv;
    if (grid > INT32_MAX) return AF_ERR_UNSUPPORTED;
    return dispatch(a, hd, n_q_heads / nkv, fp8, true, int(grid), static_cast<hipStream_t>(stream));
}
