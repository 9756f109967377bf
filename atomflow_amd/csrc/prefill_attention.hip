// prefill_attention.hip — causal GQA attention for a chunk of prompt tokens
// (prefill) over the contiguous per-layer cache, on the gfx950 matrix cores.
//
// Reference semantics: the causal kernel gqa_attention_kernel
// (src/kernel/tiled_attention.cu:34-130, launcher :136-161). Query token i of
// seq_q attends key rows s <= i, s < seq_kv (:86,:120); kv head = h*n_kv/n_q
// (:55); scores q.k * rsqrt(head_dim) (:82-96); max-subtracted softmax (:101-116);
// fp32 accumulation of p*V (:120-125); output rounded to fp16 (:126). Here the
// chunk starts at cache position p0 (chunked prefill): query i sits at position
// p0 + i and attends rows [0, min(p0 + i + 1, kv_len)). p0 = 0 with
// kv_len = seq_kv is the reference's form (af_tiled_attention).
//
// Design: one workgroup = 128 query tokens of one Q head, 4 waves x 32 queries.
//  * S^T = K Q^T on v_mfma_f32_32x32x16_f16. The A operand is a K tile read from
//    LDS, the B operand the wave's 32 queries, held in registers for the whole
//    launch. Each lane then owns 16 of the 32 scores of one query (its partner
//    lane l^32 owns the other 16), so the softmax max and sum are in-lane work
//    plus one v_permlane32_swap.
//  * O^T += V^T P^T. P^T is the S^T accumulator rounded to fp16: within each
//    16-key step the keys are numbered with bits 2 and 3 swapped, which makes the
//    accumulator's register order the operand's k order. V is stored transposed
//    in LDS in that key order, so each V^T operand is one 16-byte LDS read.
//  * K and V^T tiles of 64 keys are double-buffered in LDS. The next tile's
//    global loads are issued before the current tile's matrix work and written to
//    LDS after it: one barrier per tile.
//  * Both LDS layouts are XOR-swizzled in 16-byte chunks, so the operand reads
//    and the tile writes spread over the banks.
//  * Softmax is online in the log2 domain with lazy rescaling: the running max
//    moves only when a tile's max exceeds it by more than 2^8, so most tiles skip
//    the O^T rescale.
//  * Workgroups are launched heaviest first (the last query tiles attend the most
//    keys); waves skip key tiles that lie wholly above their queries' diagonal.
#include <cmath>

#include "af_common.h"
#include "af_device.h"

namespace af {
namespace {

constexpr int kPfHd = 128;
constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfQueries = 32 * kPfWaves;          // query tokens per workgroup
constexpr int kPfKeys = 64;                        // keys per LDS tile
constexpr int kKTileBytes = kPfKeys * kPfHd * 2;   // K rows of 256 B
constexpr int kVTileBytes = kPfHd * kPfKeys * 2;   // V^T rows (one per d) of 128 B
constexpr float kPfLazyLog2 = 8.0f;
constexpr float kPfEmptyMax = -1e30f;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

struct PrefillArgs {
    const uint16_t* q;   // query row i at q + i*q_stride, head h at +h*head_dim
    int64_t q_stride;
    const uint16_t* k;   // cache row t at k + t*kv_stride
    const uint16_t* v;
    int64_t kv_stride;
    uint16_t* out;       // output row i at out + i*out_stride
    int64_t out_stride;
    int32_t p0;
    int32_t n;
    int32_t kv_len;
    int32_t n_q_heads;
    int32_t n_kv_heads;
    int32_t n_tiles;     // ceil(n / kPfQueries)
    float scale_log2;    // log2(e) / sqrt(head_dim)
};

// Byte offset of 16-byte chunk `chunk` (0..15) of K tile row `row`.
__device__ __forceinline__ uint32_t k_off(int row, int chunk) {
    return uint32_t(row) * 256u + 16u * uint32_t(chunk ^ (row & 15));
}
// Byte offset of 16-byte chunk `chunk` (0..7) of V^T tile row `d`.
__device__ __forceinline__ uint32_t vt_off(int d, int chunk) {
    return uint32_t(d) * 128u + 16u * uint32_t(chunk ^ ((d ^ (d >> 3)) & 7));
}

__device__ __forceinline__ uint32_t word(const uint4& u, int p) {
    return p == 0 ? u.x : p == 1 ? u.y : p == 2 ? u.z : u.w;
}

// One 64-key tile in flight: thread (c = tid/16, e = tid%16) holds keys
// key0 + 4c .. +3, elements 8e .. 8e+7 of the head, for K and V. Named fields,
// not arrays: an array here is promoted to LDS by the compiler, which then
// waits for the loads right after issuing them.
struct TileRegs {
    uint4 k0, k1, k2, k3;
    uint4 v0, v1, v2, v3;
};

__device__ __forceinline__ uint4 ld16(const uint16_t* p) {
    return *reinterpret_cast<const uint4*>(p);
}

__device__ __forceinline__ void load_tile(const uint16_t* kb, const uint16_t* vb,
                                          int64_t kv_stride, int key0, int kv_len, int c, int e,
                                          TileRegs& t) {
    // Rows past kv_len load row kv_len-1: finite data whose scores are masked.
    const int r = key0 + 4 * c;
    const size_t o0 = size_t(min(r, kv_len - 1)) * kv_stride + 8 * e;
    const size_t o1 = size_t(min(r + 1, kv_len - 1)) * kv_stride + 8 * e;
    const size_t o2 = size_t(min(r + 2, kv_len - 1)) * kv_stride + 8 * e;
    const size_t o3 = size_t(min(r + 3, kv_len - 1)) * kv_stride + 8 * e;
    t.k0 = ld16(kb + o0);
    t.k1 = ld16(kb + o1);
    t.k2 = ld16(kb + o2);
    t.k3 = ld16(kb + o3);
    t.v0 = ld16(vb + o0);
    t.v1 = ld16(vb + o1);
    t.v2 = ld16(vb + o2);
    t.v3 = ld16(vb + o3);
}

__device__ __forceinline__ void store_tile(char* ks, char* vs, int c, int e, const TileRegs& t) {
    *reinterpret_cast<uint4*>(ks + k_off(4 * c + 0, e)) = t.k0;
    *reinterpret_cast<uint4*>(ks + k_off(4 * c + 1, e)) = t.k1;
    *reinterpret_cast<uint4*>(ks + k_off(4 * c + 2, e)) = t.k2;
    *reinterpret_cast<uint4*>(ks + k_off(4 * c + 3, e)) = t.k3;
    // Keys 4c..4c+3 sit in 16-key step j = c/4 at offsets 4a..4a+3 (a = c%4);
    // with bits 2 and 3 of the offset swapped they become the four consecutive
    // slots 4*sa .. 4*sa+3 of that step.
    const int j = c >> 2, a = c & 3;
    const int sa = ((a & 1) << 1) | (a >> 1);
    const int chunk = 2 * j + (sa >> 1);
    const uint32_t half_off = 8u * uint32_t(sa & 1);
    // Lanes with odd e walk their eight d rows in the order i^1, which spreads a
    // write instruction over both 128-byte halves of the bank space.
    const uint32_t sel_even = (e & 1) ? 0x07060302u : 0x05040100u;
    const uint32_t sel_odd = (e & 1) ? 0x05040100u : 0x07060302u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int p = i >> 1;
        const uint32_t sel = (i & 1) ? sel_odd : sel_even;
        uint2 pk;
        pk.x = __builtin_amdgcn_perm(word(t.v1, p), word(t.v0, p), sel);
        pk.y = __builtin_amdgcn_perm(word(t.v3, p), word(t.v2, p), sel);
        const int d = 8 * e + (i ^ (e & 1));
        *reinterpret_cast<uint2*>(vs + vt_off(d, chunk) + half_off) = pk;
    }
}

__device__ __forceinline__ half8 lds_half8(const char* p) {
    return __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(p));
}

// Max / sum over the two 32-lane halves (lane l and l^32).
__device__ __forceinline__ float halves_max(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    swap32(a, b);
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ __forceinline__ float halves_sum(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    swap32(a, b);
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

__device__ __forceinline__ half8 to_half8(const float16v& s, int base) {
    half8 h;
#pragma unroll
    for (int t = 0; t < 8; ++t) h[t] = f16(s[base + t]);
    return h;
}

__global__ __launch_bounds__(kPfThreads, 2) void prefill_attention_kernel(const PrefillArgs a) {
    __shared__ __align__(16) char s_k[2][kKTileBytes];
    __shared__ __align__(16) char s_v[2][kVTileBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform branches below
    const int col = lane & 31, hi = lane >> 5;
    const int tile = a.n_tiles - 1 - int(blockIdx.x) / a.n_q_heads;  // heaviest first
    const int head = int(blockIdx.x) % a.n_q_heads;
    const int kvh = head * a.n_kv_heads / a.n_q_heads;
    const int t0 = tile * kPfQueries;
    const int wq0 = t0 + 32 * wave;                // the wave's first query
    const bool wave_live = wq0 < a.n;
    const int qi = min(wq0 + col, a.n - 1);        // this lane's query (clamped)
    const int lim = min(a.p0 + qi + 1, a.kv_len);  // its keys: [0, lim)

    const int wg_keys = min(a.p0 + min(t0 + kPfQueries, a.n), a.kv_len);
    const int n_kt = (wg_keys + kPfKeys - 1) / kPfKeys;
    // Keys the wave needs, and the first key hidden from some of its queries.
    const int w_keys = wave_live ? min(a.p0 + min(wq0 + 32, a.n), a.kv_len) : 0;
    const int w_mask_from = min(a.p0 + wq0 + 1, a.kv_len);

    // Query operand first: the loop's first waits then cover it.
    half8 qf[8];
    {
        const uint16_t* qrow = a.q + size_t(qi) * a.q_stride + size_t(head) * kPfHd + 8 * hi;
#pragma unroll
        for (int s = 0; s < 8; ++s) qf[s] = __builtin_bit_cast(half8, ld16(qrow + 16 * s));
    }
    // Keep the query loads ahead of the tile loads: the prologue's wait for the
    // tile then covers them, and the loop never waits on a query register.
    asm volatile("" ::: "memory");
    const uint16_t* kb = a.k + size_t(kvh) * kPfHd;
    const uint16_t* vb = a.v + size_t(kvh) * kPfHd;
    const int c = tid >> 4, e = tid & 15;
    TileRegs tr;
    load_tile(kb, vb, a.kv_stride, 0, a.kv_len, c, e, tr);
    store_tile(s_k[0], s_v[0], c, e, tr);

    float16v o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    float m_run = kPfEmptyMax, l_run = 0.0f;
    const float sc = a.scale_log2;

    for (int kt = 0; kt < n_kt; ++kt) {
        __syncthreads();
        const int buf = kt & 1;
        const bool more = kt + 1 < n_kt;
        if (more) load_tile(kb, vb, a.kv_stride, (kt + 1) * kPfKeys, a.kv_len, c, e, tr);
        const int key0 = kt * kPfKeys;
        if (key0 < w_keys) {
            const char* ks = s_k[buf];
            float16v s0, s1;
#pragma unroll
            for (int r = 0; r < 16; ++r) s0[r] = s1[r] = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const half8 k0 = lds_half8(ks + k_off(col, 2 * s + hi));
                const half8 k1 = lds_half8(ks + k_off(32 + col, 2 * s + hi));
                s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(k0, qf[s], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(k1, qf[s], s1, 0, 0, 0);
            }
            // Register r of block b holds key key0 + 32b + 8(r/4) + 4hi + r%4.
            if (key0 + kPfKeys > w_mask_from) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = key0 + 8 * (r >> 2) + 4 * hi + (r & 3);
                    s0[r] = key < lim ? s0[r] : -INFINITY;
                    s1[r] = key + 32 < lim ? s1[r] : -INFINITY;
                }
            }
            float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
            for (int r = 1; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
            mx = halves_max(mx) * sc;
            const bool need = mx > m_run + kPfLazyLog2;
            if (__builtin_amdgcn_ballot_w64(need)) {
                const float m_new = need ? mx : m_run;
                const float alpha = fast_exp2(m_run - m_new);
                m_run = m_new;
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
            }
            float ls = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s0[r] = fast_exp2(fmaf(s0[r], sc, -m_run));
                s1[r] = fast_exp2(fmaf(s1[r], sc, -m_run));
                ls += s0[r] + s1[r];
            }
            l_run += ls;
            half8 pj[4];
            pj[0] = to_half8(s0, 0);
            pj[1] = to_half8(s0, 8);
            pj[2] = to_half8(s1, 0);
            pj[3] = to_half8(s1, 8);
            const char* vs = s_v[buf];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const half8 vt = lds_half8(vs + vt_off(32 * db + col, 2 * j + hi));
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vt, pj[j], o[db], 0, 0, 0);
                }
        }
        if (more) store_tile(s_k[buf ^ 1], s_v[buf ^ 1], c, e, tr);
    }

    if (!wave_live || wq0 + col >= a.n) return;
    const float inv = 1.0f / halves_sum(l_run);
    uint16_t* orow = a.out + size_t(wq0 + col) * a.out_stride + size_t(head) * kPfHd + 4 * hi;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint2 w;
            w.x = uint32_t(f2h(o[db][4 * g] * inv)) | (uint32_t(f2h(o[db][4 * g + 1] * inv)) << 16);
            w.y = uint32_t(f2h(o[db][4 * g + 2] * inv)) |
                  (uint32_t(f2h(o[db][4 * g + 3] * inv)) << 16);
            *reinterpret_cast<uint2*>(orow + 32 * db + 8 * g) = w;
        }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_prefill(const PrefillArgs& a, hipStream_t stream) {
    const int grid = a.n_tiles * a.n_q_heads;
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(grid), dim3(kPfThreads), 0, stream, a);
    AF_TRY_LAUNCH();
    return AF_OK;
}

}  // namespace
}  // namespace af

using namespace af;

// ---- b2 -----------------------------------------------------------------------
extern "C" int af_prefill_attention(const void* q, int q_stride, const void* k_cache,
                                    const void* v_cache, void* out, int out_stride, int p0, int n,
                                    int kv_len, int max_seq, int n_q_heads, int n_kv_heads,
                                    int head_dim, af_stream_t stream) {
    if (!q || !k_cache || !v_cache || !out || n < 0 || p0 < 0 || n_q_heads <= 0 ||
        n_kv_heads <= 0 || n_q_heads % n_kv_heads || max_seq <= 0)
        return AF_ERR_INVALID_ARG;
    if (head_dim != kPfHd) return AF_ERR_UNSUPPORTED;
    const int q_dim = n_q_heads * head_dim;
    if (q_stride < q_dim || out_stride < q_dim || q_stride % 8 || out_stride % 8)
        return AF_ERR_INVALID_ARG;
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
        return AF_ERR_INVALID_ARG;
    if (n == 0) return AF_OK;
    if (kv_len <= 0 || kv_len > max_seq) return AF_ERR_OUT_OF_RANGE;
    PrefillArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.q_stride = q_stride;
    a.k = static_cast<const uint16_t*>(k_cache);
    a.v = static_cast<const uint16_t*>(v_cache);
    a.kv_stride = int64_t(n_kv_heads) * head_dim;
    a.out = static_cast<uint16_t*>(out);
    a.out_stride = out_stride;
    a.p0 = p0;
    a.n = n;
    a.kv_len = kv_len;
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = n_kv_heads;
    a.n_tiles = ceil_div(n, kPfQueries);
    a.scale_log2 = float(1.4426950408889634 / std::sqrt(double(head_dim)));
    return launch_prefill(a, static_cast<hipStream_t>(stream));
}

extern "C" int af_tiled_attention(const void* q, const void* k, const void* v, void* out,
                                  int seq_q, int seq_kv, int head_dim, int n_q_heads,
                                  int n_kv_heads, af_stream_t stream) {
    if (!q || !k || !v || !out || seq_q < 0 || seq_kv < 0 || n_q_heads <= 0 || n_kv_heads <= 0)
        return AF_ERR_INVALID_ARG;
    if (head_dim != kPfHd) return AF_ERR_UNSUPPORTED;
    if (seq_q == 0) return AF_OK;
    const int q_dim = n_q_heads * head_dim;
    if (seq_kv == 0) {
        // No keys: the reference's accumulator stays 0 for every output element.
        if (!aligned16(out)) return AF_ERR_INVALID_ARG;
        return fill_u32(out, 0u, size_t(seq_q) * q_dim / 2, static_cast<hipStream_t>(stream));
    }
    return af_prefill_attention(q, q_dim, k, v, out, q_dim, 0, seq_q, seq_kv, seq_kv, n_q_heads,
                                n_kv_heads, head_dim, stream);
}
