// gemv.hip — W8A16 GEMV (FP8 E4M3 weights with fp16 group scales, fp16
// activations) and the fused decode QKV projection + RoPE + KV append, gfx950.
//
// y[n] = sum_k e4m3(W[n, k]) * scale[n, k / group] * x[k]   (the reference's
// w8a16_gemv_kernel, src/kernel/qkv_gemm.cu:32-110), fp32 accumulation, fp16
// output. M = 1: every weight byte is read once, so the roofline is HBM.
//
// Design:
//  * One wave owns RPW (1..5) rows: one row per wave up to four waves per SIMD
//    of the device, two up to sixteen (more waves in flight beat sharing the
//    activation loads over more rows). A weight row is read in 1 KB chunks, 16
//    bytes per lane (global_load_dwordx4); the activation slice of a chunk is
//    loaded once and shared by the wave's rows. All of a pass's loads (NCH
//    chunks x RPW rows; one pass for K up to 8 KB) are issued before any is used.
//  * E4M3 -> fp16 is exact (v_cvt_scalef32_pk_f16_fp8, scale 1), the product of
//    two fp16 values is exact in fp32, so each 16-element slice is summed with
//    v_dot2c_f32_f16 in fp32 and scaled once by its group scale.
//  * Lane partials are summed with DPP and v_permlane16/32_swap (no LDS).
//  * The fused QKV kernel gives each wave one rotation pair (d, d+HD/2) of one
//    head, so RoPE and the KV append run on the rounded fp16 results in
//    registers: the output equals af_w8a16_gemv followed by af_rope_append bit
//    for bit (a row's arithmetic does not depend on which wave computes it or
//    on the chunks per pass). The position and cos / sin loads go out with the
//    weight loads. The same kernel appends one token to a paged pool (fp16 or
//    FP8), the single-token form of af_paged_qkv_rope_append.
#include <algorithm>
#include <cmath>

#include "af_common.h"
#include "af_device.h"

namespace af {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kGemvWaves = 4;                 // plain GEMV: waves per workgroup
constexpr int kGemvThreads = kGemvWaves * 64;
constexpr int kQkvWaves = 5;                  // fused QKV: waves per workgroup
constexpr int kQkvPairs = 1;                  // fused QKV: rotation pairs per wave
constexpr int kQkvThreads = kQkvWaves * 64;
constexpr int kChunkBytes = 64 * 16;          // one weight-row chunk per wave load

// sum_i e4m3(w_i) * x_i over the 16 codes of `w` and 16 fp16 activations.
__device__ __forceinline__ float dot16(const uint4 w, const uint4 xa, const uint4 xb) {
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
    const uint32_t xx[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2_t w01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(ww[i]), 1.0f, false);
        const half2_t w23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(ww[i]), 1.0f, true);
        acc = __builtin_amdgcn_fdot2(w01, __builtin_bit_cast(half2_t, xx[2 * i]), acc, false);
        acc = __builtin_amdgcn_fdot2(w23, __builtin_bit_cast(half2_t, xx[2 * i + 1]), acc, false);
    }
    return acc;
}

// Lane partials of rows[r] (r < RPW) over the whole K dimension, NCH chunks
// per pass. Chunks past K are read at a clamped address and contribute 0.
// `hook` runs once, right after the first pass's loads are issued: loads the
// caller needs only after the sums (the fused kernel's position and cos / sin)
// then travel with the weight loads instead of after them.
// Weight bytes are read once per launch: non-temporal 16-B loads (the
// streaming cache policy; the activation, read by every workgroup, keeps the
// default one). NT = false: the default policy, for small matrices.
template <bool NT>
__device__ __forceinline__ uint4 load_w16(const uint8_t* p) {
    if constexpr (NT) {
        typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
        const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *reinterpret_cast<const uint4*>(p);
    }
}

struct NoHook {
    __device__ void operator()() const {}
};

template <int RPW, int NCH, typename Hook = NoHook, bool NT = true>
__device__ __forceinline__ void row_partials(const uint8_t* __restrict__ w,
                                             const uint16_t* __restrict__ x,
                                             const uint16_t* __restrict__ scales,
                                             const int (&rows)[RPW], int k, int group_size,
                                             int groups, int lane, float (&acc)[RPW],
                                             const Hook& hook = Hook()) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.f;
    for (int base = 0; base < k; base += NCH * kChunkBytes) {
        uint4 xa[NCH], xb[NCH], wv[NCH][RPW];
        uint16_t sc[NCH][RPW];
        bool in[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int k0 = base + c * kChunkBytes + lane * 16;
            in[c] = k0 < k;
            const int kk = in[c] ? k0 : 0;
            xa[c] = *reinterpret_cast<const uint4*>(x + kk);
            xb[c] = *reinterpret_cast<const uint4*>(x + kk + 8);
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                wv[c][r] = load_w16<NT>(w + size_t(rows[r]) * k + kk);
                sc[c][r] = scales[size_t(rows[r]) * groups + kk / group_size];
            }
        }
        if (base == 0) hook();
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const float part = dot16(wv[c][r], xa[c], xb[c]);
                acc[r] = in[c] ? fmaf(h2f(sc[c][r]), part, acc[r]) : acc[r];
            }
    }
}

// ---- plain GEMV: wave w of block b owns rows (4b + w) * RPW .. + RPW - 1 ----
// RPW from rows_per_wave, NCH so one pass covers K for the usual widths, NT
// the weight-load policy.
template <int RPW, int NCH, bool NT>
__global__ __launch_bounds__(kGemvThreads) void w8a16_gemv_kernel(
    const uint8_t* __restrict__ w, const uint16_t* __restrict__ x,
    const uint16_t* __restrict__ scales, uint16_t* __restrict__ y, int n, int k, int group_size) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kGemvWaves + wave) * RPW;
    if (row0 >= n) return;
    int rows[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) rows[r] = min(row0 + r, n - 1);
    float acc[RPW];
    row_partials<RPW, NCH, NoHook, NT>(w, x, scales, rows, k, group_size, k / group_size, lane,
                                       acc);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const float tot = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < n) y[row0 + r] = f2h(tot);
    }
}

// ---- two GEMVs of one activation in one launch (gate and up) -----------------
// Blocks [0, blocks0) compute matrix 0, the rest matrix 1, with the plain
// kernel's row mapping inside each: a row's arithmetic is the same as in
// w8a16_gemv_kernel, so each output equals af_w8a16_gemv bit for bit.
struct GemvPair {
    const uint8_t* w[2];
    const uint16_t* scales[2];
    uint16_t* y[2];
    int n[2];
    int blocks0;
};

template <int RPW, int NCH>
__global__ __launch_bounds__(kGemvThreads) void w8a16_gemv_pair_kernel(
    const GemvPair p, const uint16_t* __restrict__ x, int k, int group_size) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m = int(blockIdx.x) >= p.blocks0 ? 1 : 0;
    const int blk = int(blockIdx.x) - m * p.blocks0;
    const int n = p.n[m];
    const int row0 = (blk * kGemvWaves + wave) * RPW;
    if (row0 >= n) return;
    int rows[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) rows[r] = min(row0 + r, n - 1);
    float acc[RPW];
    row_partials<RPW, NCH>(p.w[m], x, p.scales[m], rows, k, group_size, k / group_size, lane, acc);
    uint16_t* y = p.y[m];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const float tot = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < n) y[row0 + r] = f2h(tot);
    }
}

// ---- fused decode QKV projection + RoPE + KV append --------------------------
// Output rows of qkv_out = [Q heads | K heads | V heads] x head_dim. Rotation
// pairs are numbered p = head * HD/2 + d; wave w of block b takes the PPW pairs
// PPW(b*kQkvWaves + w) .. + PPW - 1 of one head, i.e. rows (head, d .. d+PPW-1)
// and their partners + HD/2. DEST selects where K and V go (QkvSingleArgs).
template <int PPW, int NCH, int DEST>
__global__ __launch_bounds__(kQkvThreads) void qkv_rope_append_kernel(const QkvSingleArgs a) {
    constexpr int R = 2 * PPW;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hd = a.head_dim, half = hd / 2;
    const int n_pairs = (a.n_q_heads + 2 * a.n_kv_heads) * half;
    const int p0 = PPW * (blockIdx.x * kQkvWaves + wave);
    if (p0 >= n_pairs) return;  // half % PPW == 0: the wave's pairs are in one head
    const int head = p0 / half;
    const int dA = p0 % half;  // pairs (dA + j, dA + j + half), j < PPW
    int rows[R];
#pragma unroll
    for (int j = 0; j < PPW; ++j) {
        rows[j] = head * hd + dA + j;
        rows[PPW + j] = head * hd + dA + j + half;
    }
    // The position, the destination row and the cos / sin are read while the
    // weight loads are in flight (the table row clamped into the table).
    const bool rotate = head < a.n_q_heads + a.n_kv_heads;  // Q and K rows
    int pos = 0;
    int64_t row = 0;
    float cs[PPW], sn[PPW];
    auto fetch = [&]() {
        pos = a.d_pos ? *a.d_pos : a.pos_host;
        row = DEST == kQkvContiguous ? int64_t(pos) : *a.d_slot;
        const size_t at = size_t(min(max(pos, 0), a.max_pos - 1)) * half + dA;
#pragma unroll
        for (int j = 0; j < PPW; ++j) {
            cs[j] = rotate ? a.cos_t[at + j] : 0.f;
            sn[j] = rotate ? a.sin_t[at + j] : 0.f;
        }
    };
    float acc[R];
    row_partials<R, NCH>(a.w, a.x, a.scales, rows, a.k, a.group_size, a.k / a.group_size, lane,
                         acc, fetch);
    uint16_t out[R];
#pragma unroll
    for (int r = 0; r < R; ++r) out[r] = f2h(wave_sum(acc[r]));
    const bool ok = pos >= 0 && pos < a.max_pos && row >= 0 && row < a.max_rows;
    if (!ok && blockIdx.x == 0 && threadIdx.x == 0 && a.d_status)
        *a.d_status = AF_ERR_OUT_OF_RANGE;
    // Out of range: the contiguous form writes nothing, the paged form leaves
    // the unrotated projection in qkv_out and nothing in the pool.
    if ((!ok && DEST == kQkvContiguous) || lane != 0) return;
    if (ok && rotate) {
#pragma unroll
        for (int j = 0; j < PPW; ++j)  // the reference's rope_kernel arithmetic, rope.cu:30-45
            rope_rotate(out[j], out[PPW + j], cs[j], sn[j], out[j], out[PPW + j]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) a.qkv[rows[r]] = out[r];
    if (!ok || head < a.n_q_heads) return;
    const bool is_k = head < a.n_q_heads + a.n_kv_heads;
    const int hk = head - a.n_q_heads - (is_k ? 0 : a.n_kv_heads);
    const size_t at = size_t(row) * (a.n_kv_heads * hd) + size_t(hk) * hd + dA;
    if constexpr (DEST == kQkvPagedFp8) {
        const float sc = (is_k ? a.k_scales : a.v_scales)[hk];
        uint8_t* dst = (is_k ? a.k_dst : a.v_dst) + at;
#pragma unroll
        for (int j = 0; j < PPW; ++j) {
            dst[j] = uint8_t(quantize_fp8(out[j], sc));
            dst[j + half] = uint8_t(quantize_fp8(out[PPW + j], sc));
        }
    } else {
        uint16_t* dst = reinterpret_cast<uint16_t*>(is_k ? a.k_dst : a.v_dst) + at;
#pragma unroll
        for (int j = 0; j < PPW; ++j) {
            dst[j] = out[j];
            dst[j + half] = out[PPW + j];
        }
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_gemv_shape(const void* x, const uint8_t* w, const void* scales, int n, int k,
                     int group_size) {
    if (!x || !w || !scales || n <= 0 || k <= 0 || group_size <= 0) return AF_ERR_INVALID_ARG;
    if (k % 16 || group_size % 16 || k % group_size) return AF_ERR_UNSUPPORTED;
    if (!aligned16(x) || !aligned16(w)) return AF_ERR_INVALID_ARG;
    return AF_OK;
}

// Chunks per pass: all of K in one pass for the usual widths.
int chunks_per_pass(int k) {
    if (k == 3 * kChunkBytes || k == 6 * kChunkBytes) return 3;
    if (k > 4 * kChunkBytes && k <= 8 * kChunkBytes) return 8;
    return 4;
}

// Weight matrices from this size on stream with non-temporal loads; smaller
// ones measured faster with the default policy (o_proj 3072 x 3072, 9.4 MB:
// 4.04 against 4.12 us; the 15.7 MB QKV projection 5.58 against 5.04 us).
constexpr size_t kStreamWeightBytes = size_t(12) << 20;

template <int RPW, bool NT>
void launch_gemv_policy(int nch, hipStream_t s, const uint8_t* w, const uint16_t* x,
                        const uint16_t* sc, uint16_t* y, int n, int k, int group_size) {
    const int grid = (n + kGemvWaves * RPW - 1) / (kGemvWaves * RPW);
    if (nch == 3)
        hipLaunchKernelGGL((w8a16_gemv_kernel<RPW, 3, NT>), dim3(grid), dim3(kGemvThreads), 0, s, w,
                           x, sc, y, n, k, group_size);
    else if (nch == 8)
        hipLaunchKernelGGL((w8a16_gemv_kernel<RPW, 8, NT>), dim3(grid), dim3(kGemvThreads), 0, s, w,
                           x, sc, y, n, k, group_size);
    else
        hipLaunchKernelGGL((w8a16_gemv_kernel<RPW, 4, NT>), dim3(grid), dim3(kGemvThreads), 0, s, w,
                           x, sc, y, n, k, group_size);
}

template <int RPW>
void launch_gemv(int nch, hipStream_t s, const uint8_t* w, const uint16_t* x, const uint16_t* sc,
                 uint16_t* y, int n, int k, int group_size) {
    if (size_t(n) * size_t(k) >= kStreamWeightBytes)
        launch_gemv_policy<RPW, true>(nch, s, w, x, sc, y, n, k, group_size);
    else
        launch_gemv_policy<RPW, false>(nch, s, w, x, sc, y, n, k, group_size);
}

// Rows per wave for n rows: 1 up to four waves per SIMD, 2 up to sixteen, then
// as many as keep eight waves per SIMD (at most 5). Measured on the Llama-3.2-3B
// shapes (3072 / 8192 / 16384 rows): fewer rows per wave, and so more waves with
// loads in flight, is faster until the activation loads (one per row at RPW 1)
// cost more than the extra waves win.
int rows_per_wave(int n) {
    const int simds = 4 * device_compute_units();
    return n <= 4 * simds ? 1 : (n <= 16 * simds ? 2 : std::min(5, (n + 8 * simds - 1) / (8 * simds)));
}

template <int RPW, int NCH>
void launch_pair_nch(const GemvPair& p, const uint16_t* x, int k, int group_size, hipStream_t s) {
    const int per_block = kGemvWaves * RPW;
    GemvPair q = p;
    q.blocks0 = (p.n[0] + per_block - 1) / per_block;
    const int grid = q.blocks0 + (p.n[1] + per_block - 1) / per_block;
    hipLaunchKernelGGL((w8a16_gemv_pair_kernel<RPW, NCH>), dim3(grid), dim3(kGemvThreads), 0, s,
                       q, x, k, group_size);
}

template <int RPW>
void launch_pair(int nch, const GemvPair& p, const uint16_t* x, int k, int group_size,
                 hipStream_t s) {
    if (nch == 3)
        launch_pair_nch<RPW, 3>(p, x, k, group_size, s);
    else if (nch == 8)
        launch_pair_nch<RPW, 8>(p, x, k, group_size, s);
    else
        launch_pair_nch<RPW, 4>(p, x, k, group_size, s);
}

template <int PPW, int NCH>
void launch_qkv_nch(const QkvSingleArgs& q, int dest, hipStream_t s) {
    const int n_pairs = (q.n_q_heads + 2 * q.n_kv_heads) * (q.head_dim / 2);
    const dim3 grid((n_pairs + PPW * kQkvWaves - 1) / (PPW * kQkvWaves));
    if (dest == kQkvPagedFp8)
        hipLaunchKernelGGL((qkv_rope_append_kernel<PPW, NCH, kQkvPagedFp8>), grid,
                           dim3(kQkvThreads), 0, s, q);
    else if (dest == kQkvPagedFp16)
        hipLaunchKernelGGL((qkv_rope_append_kernel<PPW, NCH, kQkvPagedFp16>), grid,
                           dim3(kQkvThreads), 0, s, q);
    else
        hipLaunchKernelGGL((qkv_rope_append_kernel<PPW, NCH, kQkvContiguous>), grid,
                           dim3(kQkvThreads), 0, s, q);
}

}  // namespace

void launch_qkv_single(const QkvSingleArgs& q, int dest, hipStream_t s) {
    const int nch = chunks_per_pass(q.k);
    if (nch == 3)
        launch_qkv_nch<kQkvPairs, 3>(q, dest, s);
    else if (nch == 8)
        launch_qkv_nch<kQkvPairs, 8>(q, dest, s);
    else
        launch_qkv_nch<kQkvPairs, 4>(q, dest, s);
}

}  // namespace af

using namespace af;

extern "C" int af_w8a16_gemv_pair(const void* x, const uint8_t* weight0, const void* scales0,
                                  void* y0, int n0, const uint8_t* weight1, const void* scales1,
                                  void* y1, int n1, int k, int group_size, af_stream_t stream) {
    if (int st = check_gemv_shape(x, weight0, scales0, n0, k, group_size)) return st;
    if (int st = check_gemv_shape(x, weight1, scales1, n1, k, group_size)) return st;
    if (!y0 || !y1) return AF_ERR_INVALID_ARG;
    GemvPair p;
    p.w[0] = weight0;
    p.w[1] = weight1;
    p.scales[0] = static_cast<const uint16_t*>(scales0);
    p.scales[1] = static_cast<const uint16_t*>(scales1);
    p.y[0] = static_cast<uint16_t*>(y0);
    p.y[1] = static_cast<uint16_t*>(y1);
    p.n[0] = n0;
    p.n[1] = n1;
    p.blocks0 = 0;
    const int nch = chunks_per_pass(k);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const auto* xw = static_cast<const uint16_t*>(x);
    switch (rows_per_wave(n0 + n1)) {
        case 1: launch_pair<1>(nch, p, xw, k, group_size, s); break;
        case 2: launch_pair<2>(nch, p, xw, k, group_size, s); break;
        case 3: launch_pair<3>(nch, p, xw, k, group_size, s); break;
        case 4: launch_pair<4>(nch, p, xw, k, group_size, s); break;
        default: launch_pair<5>(nch, p, xw, k, group_size, s); break;
    }
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" int af_w8a16_gemv(const void* x, const uint8_t* weight, const void* scales, void* y,
                             int n, int k, int group_size, af_stream_t stream) {
    if (int st = check_gemv_shape(x, weight, scales, n, k, group_size)) return st;
    if (!y) return AF_ERR_INVALID_ARG;
    const int rpw = rows_per_wave(n);
    const int nch = chunks_per_pass(k);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const auto* xw = static_cast<const uint16_t*>(x);
    const auto* sw = static_cast<const uint16_t*>(scales);
    auto* yw = static_cast<uint16_t*>(y);
    switch (rpw) {
        case 1: launch_gemv<1>(nch, s, weight, xw, sw, yw, n, k, group_size); break;
        case 2: launch_gemv<2>(nch, s, weight, xw, sw, yw, n, k, group_size); break;
        case 3: launch_gemv<3>(nch, s, weight, xw, sw, yw, n, k, group_size); break;
        case 4: launch_gemv<4>(nch, s, weight, xw, sw, yw, n, k, group_size); break;
        default: launch_gemv<5>(nch, s, weight, xw, sw, yw, n, k, group_size); break;
    }
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" int af_qkv_rope_append(const void* x, const uint8_t* w_qkv, const void* scales, int k,
                                  int group_size, void* qkv_out, void* k_cache, void* v_cache,
                                  const float* cos_table, const float* sin_table, int pos,
                                  const int32_t* d_pos, int max_seq, int n_q_heads,
                                  int n_kv_heads, int head_dim, int32_t* d_status,
                                  af_stream_t stream) {
    if (n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0) return AF_ERR_INVALID_ARG;
    const int n = (n_q_heads + 2 * n_kv_heads) * head_dim;
    if (int st = check_gemv_shape(x, w_qkv, scales, n, k, group_size)) return st;
    if (!qkv_out || !k_cache || !v_cache || !cos_table || !sin_table || max_seq <= 0)
        return AF_ERR_INVALID_ARG;
    if (head_dim % 2) return AF_ERR_UNSUPPORTED;  // rotation pairs (d, d + head_dim / 2)
    if (!d_pos && (pos < 0 || pos >= max_seq)) return AF_ERR_OUT_OF_RANGE;
    QkvSingleArgs q{};
    q.w = w_qkv;
    q.x = static_cast<const uint16_t*>(x);
    q.scales = static_cast<const uint16_t*>(scales);
    q.k = k;
    q.group_size = group_size;
    q.qkv = static_cast<uint16_t*>(qkv_out);
    q.k_dst = static_cast<uint8_t*>(k_cache);
    q.v_dst = static_cast<uint8_t*>(v_cache);
    q.cos_t = cos_table;
    q.sin_t = sin_table;
    q.pos_host = pos;
    q.d_pos = d_pos;
    q.max_pos = max_seq;
    q.max_rows = max_seq;
    q.n_q_heads = n_q_heads;
    q.n_kv_heads = n_kv_heads;
    q.head_dim = head_dim;
    q.d_status = d_status;
    launch_qkv_single(q, kQkvContiguous, static_cast<hipStream_t>(stream));
    AF_TRY_LAUNCH();
    return AF_OK;
}
