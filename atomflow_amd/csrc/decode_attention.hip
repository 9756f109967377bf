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
//    one): every load instruction reads whole 128-B lines. FP8 workgroups take
//    a pair of KV heads (lanes 0-7 of a 16-lane row one head, 8-15 the next),
//    so each row read is 256 contiguous bytes: 128-B pieces 1 KB apart stream
//    at ~0.66 of HBM peak on MI355X, 256-B pieces at ~0.75. QK partial dots are
//    summed across the 8 lanes with three DPP adds; the softmax max is made
//    wave-uniform per chunk so the accumulator rescale is a uniform branch.
//  * fp32 online softmax (exp2 with log2(e) folded into the score scale), fp32
//    accumulation via v_fma_mix (fp16 V) or v_cvt_pk_f32_fp8 (FP8 V).
//  * The last workgroup of a (sequence, KV head) to finish merges the splits'
//    (m, l, o[]) partials and writes fp16 output; it also re-zeroes the arrival
//    counter, so the kernel is one launch and replays inside a hipGraph.
//  * Paged: the split's block-table entries are staged in LDS once; rows are
//    addressed block * block_size + (t mod block_size) within the layer slab.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>
#include <vector>

#include "af_common.h"
#include "af_device.h"

namespace af {
namespace {

#ifdef AF_PHASE_STAMPS
// Measurement build only (`make stamps`, libatomflow_kv_stamps.so): thread 0
// of every workgroup records s_memrealtime (100 MHz) at each phase of the
// decode kernel; af_dbg_phase_stamps copies the table out. Split phases: 0
// start, 1 ring prologue issued, 2 main loop entered, 3 rows streamed, 4
// partials in LDS, 5 partial stores issued, 6 stores acknowledged (flag set).
// Dedicated-combiner phases: 0 start, 6 last flag seen, 7 output written.
// Grid and dedicated-combiner forms also record 8 kernel entry (before the
// split mapping) with, in slot 9, the hardware ids XCC_ID | HW_ID << 32 (CU,
// shader array and engine; one 16-byte store), 10 last-arrival combine done,
// 11 block-table window staged (paged). Slots are not cleared: a reader keeps
// a slot only if it is later than the same workgroup's entry.
constexpr int kStampWgs = 4096, kStampPhases = 12;
__device__ __align__(16) uint64_t g_phase_stamps[kStampWgs][kStampPhases];
#define AF_STAMP(ph)                                                                       \
    do {                                                                                   \
        __builtin_amdgcn_sched_barrier(0);                                                 \
        if (threadIdx.x == 0 && blockIdx.x < kStampWgs)                                    \
            g_phase_stamps[blockIdx.x][ph] = __builtin_amdgcn_s_memrealtime();             \
        __builtin_amdgcn_sched_barrier(0);                                                 \
    } while (0)
#define AF_STAMP_ENTRY()                                                                   \
    do {                                                                                   \
        __builtin_amdgcn_sched_barrier(0);                                                 \
        if (threadIdx.x == 0 && blockIdx.x < kStampWgs) {                                  \
            uint32_t xcc, hwid;                                                            \
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 16)" : "=s"(xcc));      \
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hwid));             \
            const uint64_t t = __builtin_amdgcn_s_memrealtime();                           \
            *reinterpret_cast<ulonglong2*>(&g_phase_stamps[blockIdx.x][8]) =               \
                make_ulonglong2(t, uint64_t(xcc) | (uint64_t(hwid) << 32));                \
        }                                                                                  \
        __builtin_amdgcn_sched_barrier(0);                                                 \
    } while (0)
#else
#define AF_STAMP(ph) \
    do {             \
    } while (0)
#define AF_STAMP_ENTRY() \
    do {                 \
    } while (0)
#endif

typedef _Float16 f16;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;              // waves per workgroup
constexpr int kThreads = kWaves * 64;  // 256
constexpr int kLanesPerRow = 8;        // lanes that share one token row of one head
constexpr int kRowsPerStep = 64 / kLanesPerRow;      // 8 tokens per wave row-step
constexpr int kStepTokens = kWaves * kRowsPerStep;   // 32 tokens per workgroup step (one KV head)
constexpr int kMaxTableLds = 1024;     // block-table entries staged per split
constexpr int kRingBudget = 126;       // VGPRs shared by the row ring and the accumulators
constexpr float kLazyLog2 = 8.0f;      // running-max slack before a rescale (log2 units)
constexpr float kEmptyMax = -1.0e30f;  // running max of a lane group that has seen no row

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

// Sum over the 8 token groups of the lanes that share lane & 7.
__device__ __forceinline__ float groups_sum(float v) { return rows_sum(v + dpp<0x128>(v)); }

__device__ __forceinline__ int ceil_div_d(int a, int b) { return (a + b - 1) / b; }

// Agent-scope (all XCDs) relaxed atomic store / load of split-K partials.
__device__ __forceinline__ void store_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct AttnArgs {
    uint16_t* q;       // query rows; pre-RoPE qkv rows in the fused kernel
    int64_t q_stride;  // elements between sequences
    uint8_t* k;        // contiguous cache base, or the layer's K slab
    uint8_t* v;
    int64_t row_bytes;  // bytes between consecutive token rows (kv_dim * elem)
    const int32_t* tables;
    int32_t max_blocks;
    int32_t block_shift;
    int64_t total_blocks;
    const int32_t* seq_lens;  // unfused: [batch] lengths, or NULL -> seq_len_host
    int32_t seq_len_host;
    int32_t max_seq_len;      // bound on every length (rows addressable)
    // fused RoPE + append
    const int32_t* positions;  // [batch] positions, or NULL -> pos_host
    int32_t pos_host;
    const int64_t* slots;      // paged: [batch] physical rows of the new token
    int64_t max_rows;          // rows in the destination
    const float* cos_t;
    const float* sin_t;
    int32_t max_pos;           // rows in the RoPE table
    int32_t* d_status;
    // output
    uint16_t* out;
    int64_t out_stride;
    int32_t n_kv_heads;
    int32_t num_splits;
    int32_t span_tokens;  // target tokens per split: a sequence uses ceil(L / span) splits
    float qk_scale;       // log2(e) / sqrt(head_dim)
    const float* scales;  // FP8: [2][n_kv_heads] (K, V) of this layer
    float* part_o;        // [batch][n_kv_heads][rec_stride][GROUP * head_dim]
    float* part_ml;       // [batch][n_kv_heads][rec_stride][2 * GROUP]  (m..., l...)
    uint32_t* counters;   // [batch][n_kv_heads]
    // Dedicated-combiner form: workgroups [0, split_wgs) are splits, the next
    // batch * n_kv_heads are one combiner per (sequence, KV head) that waits on
    // its splits' ready flags ([batch * n_kv_heads][kCombSplits]).
    uint32_t* flags;
    int32_t split_wgs;
    int32_t batch;       // sequences (the persistent form claims items over their rows)
    int32_t item_big;    // persistent form: row-steps of a big / small item
    int32_t item_small;
    // Shared prefix: rows [0, row_start) of every sequence are covered by
    // pre_records partials already in records 0 .. pre_records-1 (written by an
    // earlier launch); the splits cover rows [row_start, L) and write records
    // pre_records + split. rec_stride = records per (sequence, KV head).
    int32_t row_start;
    int32_t pre_records;
    int32_t rec_stride;
    // Batched paged grid form (up to kThreads sequences, no shared prefix): the
    // grid is batch x heads x num_splits, but a sequence uses only the splits
    // its length needs. Workgroups then map onto the splits that exist (sequence
    // by sequence, heads fastest) and the surplus, at the end of the grid,
    // exits at once, instead of idle workgroups spread through the grid each
    // holding a slot for a length read.
    int32_t compact;
    // Paged pools with AF_KV_POOL_SHARED_BLOCKS (host side): the launch takes
    // the CACHED kernels, which read KV rows with the ordinary cache policy
    // instead of non-temporal loads.
    int32_t cached_rows;
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


// Load-policy tags of the decode kernel's row loads.
using StreamTag = std::integral_constant<bool, true>;
using DefaultTag = std::integral_constant<bool, false>;
constexpr StreamTag kStream{};
constexpr DefaultTag kDefault{};

// One 16-byte non-temporal load (`global_load_dwordx4 ... nt`).
__device__ __forceinline__ uint4 load_nt(const uint8_t* p) {
    typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t quantize_fp8_dev(uint16_t h, float scale) {
    float v = float(__builtin_bit_cast(f16, h)) / scale;
    v = fminf(fmaxf(v, -448.0f), 448.0f);
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x43e00000u) return sign | 0x7eu;
    if (a < 0x3c800000u) return sign | uint32_t(__builtin_rintf(__builtin_bit_cast(float, a) * 512.0f));
    const int e = int(a >> 23) - 127;
    const uint32_t mant = a & 0x7fffffu;
    uint32_t m3 = mant >> 20;
    const uint32_t rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) m3 += 1;
    return sign | ((uint32_t(e + 7) << 3) + m3);
}

__device__ __forceinline__ uint64_t load_agent_u64(const float* p) {
    return __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Polls of a dedicated combiner before it gives up (each waits one memory
// round trip, ~0.5 us: about a second). Reached only if a split never
// publishes; the output is then NaN and *d_status (if given) AF_ERR_TIMEOUT.
constexpr int kCombMaxPolls = 1 << 21;

// Split-K merge weights over records held one per lane (lane s: record s of a
// query head; lanes past the last record hold m = -inf, l = 0): the max M, then
// w_s = exp2(m_s - M) / sum_s exp2(m_s - M) l_s in lane s. Both merges (the
// last-arrival combine and combine_dedicated) use it, so they agree bit for bit.
__device__ __forceinline__ float merge_weight(float m, float l) {
    const float mx = wave_max(m);
    const float e = fast_exp2(m - mx);  // 0 for lanes without a record
    float ls = 0.f;
    ls += e * l;
    return e * (1.0f / wave_sum(ls));
}

// Dedicated combiner of (sequence b, KV head hw), contiguous fp16, head_dim 128:
// wave w serves query head w (64 lanes x 2 outputs; GROUP <= 4, host-checked).
// Every wave polls the n_active <= kCombSplits ready flags (lane s: split s),
// and loads a split's record as soon as its flag is set, so the records of
// splits that finish early are in registers before the last one arrives: lane s
// keeps split s's (m, l), every lane its two outputs of each split. A split sets
// its flag after its partial stores are acknowledged at agent scope (the store
// / vmcnt rules of the arrival counter below), and the flag and record loads are
// agent-scope, so a set flag means the record is readable.
template <int HD, int GROUP, bool FUSED>
__device__ __forceinline__ void combine_dedicated(const AttnArgs& a, int b, int hw, int n_active,
                                                  int pos) {
    static_assert(HD == 128 && GROUP <= kWaves, "one query head per combiner wave");
    constexpr int GQ = GROUP, GHD = GROUP * HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool act = wave < GROUP;
    const int gh = act ? wave : 0;
    const int e = gh * HD + 2 * lane;  // the lane's outputs e, e + 1
    const size_t grp = size_t(b) * a.n_kv_heads + hw;
    const float* ml = a.part_ml + grp * a.rec_stride * 2 * GQ;
    const uint64_t* po = reinterpret_cast<const uint64_t*>(a.part_o + grp * a.rec_stride * GHD);
    uint32_t* flags = a.flags + grp * kCombSplits;
    // A combiner that gave up poisons the workspace (a split that publishes
    // after that sets a flag nothing clears); every later combiner on it then
    // trusts no flag and writes NaN with AF_ERR_TIMEOUT, until the workspace
    // is re-initialised.
    uint32_t* poison = a.counters + kPoisonWord;
    const bool poisoned =
        __hip_atomic_load(poison, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;

    // The query heads are stored back rotated, as the last-arrival combine does
    // (every split has read them once the records are complete). Their inputs
    // are read now; a rotation pairs dims (d, d + HD/2), held by two lanes.
    constexpr int half = HD / 2;
    uint16_t* qh = a.q + size_t(b) * a.q_stride + size_t(hw) * GHD + size_t(gh) * HD;
    const int d = 2 * lane, dd = d % half;
    uint32_t qx = 0, qy = 0;
    float2 cs = make_float2(0.f, 0.f), sn = make_float2(0.f, 0.f);
    if constexpr (FUSED) {
        if (act) {
            qx = *reinterpret_cast<const uint32_t*>(qh + dd);
            qy = *reinterpret_cast<const uint32_t*>(qh + dd + half);
            cs = *reinterpret_cast<const float2*>(a.cos_t + size_t(pos) * half + dd);
            sn = *reinterpret_cast<const float2*>(a.sin_t + size_t(pos) * half + dd);
        }
    }

    AF_STAMP(0);
    const uint32_t all = n_active >= 32 ? ~0u : ((1u << n_active) - 1u);
    uint32_t have = 0;
    float mv = -INFINITY, lv = 0.f;  // lane s: split s
    uint64_t ov[kCombSplits];
#pragma unroll
    for (int sp = 0; sp < kCombSplits; ++sp) ov[sp] = 0;
    if (act && !poisoned) {
        for (int polls = 0; have != all && polls < kCombMaxPolls; ++polls) {
            const uint32_t f = lane < n_active ? __hip_atomic_load(flags + lane, __ATOMIC_RELAXED,
                                                                   __HIP_MEMORY_SCOPE_AGENT)
                                               : 0u;
            const uint32_t fresh = uint32_t(__builtin_amdgcn_ballot_w64(f != 0u)) & all & ~have;
            if (lane < kCombSplits && ((fresh >> lane) & 1u)) {
                mv = load_agent(ml + lane * 2 * GQ + gh);
                lv = load_agent(ml + lane * 2 * GQ + GQ + gh);
            }
#pragma unroll
            for (int sp = 0; sp < kCombSplits; ++sp)
                if ((fresh >> sp) & 1u)
                    ov[sp] = __hip_atomic_load(po + size_t(sp) * (GHD / 2) + e / 2,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            have |= fresh;
        }
    }
    const bool timed_out = act && have != all;
    AF_STAMP(6);

    const float w = merge_weight(mv, lv);  // lane s: split s's weight
    float r0 = 0.f, r1 = 0.f;
#pragma unroll
    for (int sp = 0; sp < kCombSplits; ++sp) {
        if (sp < n_active) {
            const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                           __builtin_bit_cast(uint32_t, w), sp));
            r0 = fmaf(ws, __builtin_bit_cast(float, uint32_t(ov[sp])), r0);
            r1 = fmaf(ws, __builtin_bit_cast(float, uint32_t(ov[sp] >> 32)), r1);
        }
    }
    if (timed_out) r0 = r1 = __builtin_nanf("");
    uint32_t qrot = 0;
    if (act) {
        uint16_t* out_b = a.out + size_t(b) * a.out_stride + size_t(hw) * GHD;
        const uint32_t pair = uint32_t(__builtin_bit_cast(uint16_t, f16(r0))) |
                              (uint32_t(__builtin_bit_cast(uint16_t, f16(r1))) << 16);
        *reinterpret_cast<uint32_t*>(out_b + e) = pair;
        if constexpr (FUSED) {
            const float cc[2] = {cs.x, cs.y}, ss[2] = {sn.x, sn.y};
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                uint16_t xo, yo;
                rope_rotate(uint16_t(qx >> (16 * u)), uint16_t(qy >> (16 * u)), cc[u], ss[u], xo, yo);
                qrot |= uint32_t(d < half ? xo : yo) << (16 * u);
            }
        }
    }
    AF_STAMP(7);
    if (timed_out && lane == 0) {
        __hip_atomic_store(poison, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.d_status) *a.d_status = AF_ERR_TIMEOUT;
    }
    // Every wave has read Q and finished polling past this barrier: the flags
    // return to zero for the next launch and the rotated Q is stored.
    __syncthreads();
    if (tid < n_active)
        __hip_atomic_store(flags + tid, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (FUSED)
        if (act) *reinterpret_cast<uint32_t*>(qh + d) = qrot;
}

// Exclusive prefix sums of v[0, n) into pre[0, n] (pre[n] = total), n <=
// 4 * kThreads, by the whole workgroup.
__device__ __forceinline__ void block_exclusive_scan(const int32_t* v, int64_t* pre, int n) {
    __shared__ int64_t s_wave[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int64_t x[4];
    int64_t own = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = tid * 4 + u;
        x[u] = i < n ? v[i] : 0;
        own += x[u];
    }
    int64_t inc = own;  // inclusive scan over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t y = __shfl_up(inc, d);
        if (lane >= d) inc += y;
    }
    if (lane == 63) s_wave[wave] = inc;
    __syncthreads();
    int64_t base = 0;
    for (int w = 0; w < wave; ++w) base += s_wave[w];
    int64_t run = base + inc - own;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = tid * 4 + u;
        if (i < n) pre[i] = run;
        run += x[u];
    }
    if (tid == kThreads - 1) pre[n] = run;
    __syncthreads();
}

// Splits of a sequence attending L rows in the grid form (rows of STEP per
// workgroup step): the rows after the shared prefix (all rows [0, L) when L is
// below it) in spans of about span_tokens, at least one and at most
// num_splits; an empty sequence keeps one workgroup for its zero output.
__device__ __forceinline__ int grid_splits(const AttnArgs& a, int L, int step_rows) {
    if (L <= 0) return 1;
    const bool below_prefix = L < a.row_start;
    const int t_lo = below_prefix ? 0 : min(a.row_start, L - 1);
    const int total_steps = (L - t_lo + step_rows - 1) / step_rows;
    const int span_steps = max(1, a.span_tokens / step_rows);
    return max(1, min(a.num_splits, (total_steps + span_steps - 1) / span_steps));
}

// Inclusive prefix sum over the wave's 64 lanes on DPP: row_shr 1, 2, 4, 8
// within each 16-lane row, then row_bcast 15 and 31 carry the row totals up.
__device__ __forceinline__ int wave_inclusive_sum(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false); // row_bcast:15 -> rows 1, 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false); // row_bcast:31 -> rows 2, 3
    return x;
}

// One decode-attention work item: rows [t_begin, t_end) of (sequence b, KV
// head group hw), split `split` of n_active (record slot pre_used + split).
struct Seg {
    int b, hw, split, n_active, pre_used;
    int L, pos;                 // attended rows; the appended row's position (fused)
    int t_begin, t_end, t_valid, n_steps;
    // Persistent form: this item's block-table window was loaded by the
    // previous item (thread t holds entry t).
    int staged;
};

// Streams one work item and publishes its partial (or the output when it is
// the item's only split); the last split of (b, hw) to publish merges them.
struct NoNextItem {
    __device__ bool operator()(uint32_t, int*, int*, int*) const { return false; }
};

template <int HD, int GROUP, bool FP8, bool PAGED, bool FUSED, bool PAIR, bool COMB, bool CACHED,
          bool PERSIST = false, typename NextFn = NoNextItem>
__device__ __forceinline__ void decode_attn_seg(const AttnArgs& a, const Seg& sg, int32_t& nx_entry,
                                                uint32_t next_item = 0,
                                                const NextFn& next_window = NextFn()) {
    using LY = Layout<HD, FP8>;
    constexpr int LOADS = LY::kLoads;
    constexpr int EPL = LY::kEpl;
    constexpr int KVH = PAIR ? 2 : 1;          // KV heads per workgroup
    constexpr int GQ = GROUP * KVH;            // query heads per workgroup
    constexpr int GHD = GQ * HD;               // output / record width of the workgroup
    constexpr int LANES_ROW = kLanesPerRow * KVH;
    constexpr int ROWS_WAVE = 64 / LANES_ROW;  // token rows per wave row-step
    constexpr int STEP = kWaves * ROWS_WAVE;   // token rows per workgroup step
    constexpr int kParts = PAIR ? kWaves : 4 * kWaves;  // partials per head staged in LDS
    constexpr int V16 = LY::kRowBytes / 16;    // 16-B pieces of one head's row
    // Row-steps in flight per lane: as many as fit beside the accumulators.
    constexpr int kRowRegs = 2 * LOADS * 4;
    constexpr int kFree = kRingBudget - GROUP * (EPL + EPL / 2 + 2);
    constexpr int NB_FIT = kFree / kRowRegs < 2 ? 2 : (kFree / kRowRegs > 8 ? 8 : kFree / kRowRegs);
    // FP8 consumes slots in pairs and is VALU-bound: 4 slots keep the paired
    // fused form within 3 waves per SIMD. Fused and unfused kernels use the
    // same NB, so both process the same rows in pairs (bit-identical results).
    constexpr int NB = FP8 ? (NB_FIT > 4 ? 4 : NB_FIT) : NB_FIT;

    __shared__ __align__(16) float s_acc[kParts][GHD];  // partial o of every row group / wave
    __shared__ float s_pm[kParts][GQ];
    __shared__ float s_pl[kParts][GQ];
    __shared__ int32_t s_tab[PAGED ? kMaxTableLds : 1];
    __shared__ float s_ml[2 * GQ * kMaxSplits];  // (m, l) of every split
    __shared__ __align__(16) float s_wt[GQ][kMaxSplits];
    __shared__ uint16_t s_q[FUSED ? GHD : 1];
    __shared__ uint4 s_new[FUSED ? KVH * 2 * V16 : 1];  // new token's K then V row, per KV head
    __shared__ int s_last;
    __shared__ uint32_t s_next;  // persistent form: the item claimed for after this one

    int tid = threadIdx.x;
    // The persistent form runs items in a loop: an opaque thread id keeps the
    // compiler from hoisting per-lane values out of it (they would stay live
    // across every item, past the register budget of 3 workgroups per CU).
    if constexpr (PERSIST) asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane / LANES_ROW, j = lane & 7;
    const int sub = PAIR ? (lane >> 3) & 1 : 0;  // which KV head of the pair this lane reads
    const int nkv = a.n_kv_heads;
    const int nhw = nkv / KVH;  // workgroups per (sequence, split)
    const int b = sg.b, hw = sg.hw, split = sg.split, n_active = sg.n_active;
    const int pre_used = sg.pre_used, L = sg.L, pos = sg.pos;
    const int t_begin = sg.t_begin, t_end = sg.t_end, t_valid = sg.t_valid, n_steps = sg.n_steps;
    const int h = hw * KVH + sub;  // this lane's KV head
    uint16_t* out_b = a.out + size_t(b) * a.out_stride + size_t(hw) * GHD;
    const bool direct = n_active == 1 && pre_used == 0;  // no combine: write the output
    const bool owner = FUSED && split == n_active - 1;  // holds the new token (t = L - 1)
    AF_STAMP(0);

    // ---- stage this split's block-table entries (paged) --------------------
    int tab_base = 0;
    if constexpr (PAGED) {
        const int first = t_begin >> a.block_shift;
        const int last = (t_end - 1) >> a.block_shift;
        tab_base = first;
        if (PERSIST && sg.staged) {
            // the previous item loaded this window's entries (thread t holds
            // entry t) while it merged
            if (tid <= last - first) s_tab[tid] = min(max(nx_entry, 0), int(a.total_blocks - 1));
        } else {
            const int32_t* trow = a.tables + size_t(b) * a.max_blocks;
            for (int e = tid; e <= last - first; e += kThreads) {
                int blk = trow[first + e];
                blk = min(max(blk, 0), int(a.total_blocks - 1));  // never address outside the pool
                s_tab[e] = blk;
            }
        }
        __syncthreads();
        AF_STAMP(11);
    }

    const uint8_t* kbase = a.k + size_t(h) * LY::kRowBytes + j * 16;
    const uint8_t* vbase = a.v + size_t(h) * LY::kRowBytes + j * 16;
    // Rows that may be read from memory: [t_begin, L) unfused; [t_begin, L-1)
    // fused (row L-1 is the token being appended and comes from LDS). A fused
    // split that starts at row L-1 reads row t_begin (staged, discarded): the
    // row clamp never leaves the split's staged block-table window.
    const int last_row = FUSED ? max(L - 2, t_begin) : L - 1;
    // Token of this lane in step s: waves interleave 8-row slices of each step.
    const int lane_t0 = t_begin + wave * ROWS_WAVE + g;

    struct Row {
        uint4 k[LOADS];
        uint4 v[LOADS];
    };

    auto row_offset = [&](int t) -> int64_t {
        const int tc = min(t, last_row);  // rows past the range are read in-bounds and masked
        if constexpr (PAGED) {
            const int mask = (1 << a.block_shift) - 1;
            const int64_t blk = s_tab[(tc >> a.block_shift) - tab_base];
            return ((blk << a.block_shift) | (tc & mask)) * a.row_bytes;
        } else {
            return int64_t(tc) * a.row_bytes;
        }
    };

    // KV rows are read with non-temporal loads (`nt`, the streaming cache
    // policy), since a launch reads each row once: on MI355X that measured 4-7%
    // less time per launch than the default policy, batch 1 and batched, fp16
    // and FP8. CACHED kernels (paged pools whose blocks may be mapped by
    // several sequences of a launch: forks, prefix caching) keep the default
    // policy, so that the sequences after the first find shared rows in L2
    // (64 forks of a 2048-row prefix: 68 us per launch, 85 us streaming).
    // `stream` is kStream or kDefault; kDefault takes the default policy in
    // every kernel (the paged last round's refills, whose re-reads of the
    // split's last step then hit L2).
    auto load_row = [&](Row& r, int step, auto stream) {
        const int64_t off = row_offset(lane_t0 + step * STEP);
        if constexpr (!CACHED && decltype(stream)::value) {
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                r.k[i] = load_nt(kbase + off + i * 128);
                r.v[i] = load_nt(vbase + off + i * 128);
            }
        } else {
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                r.k[i] = *reinterpret_cast<const uint4*>(kbase + off + i * 128);
                r.v[i] = *reinterpret_cast<const uint4*>(vbase + off + i * 128);
            }
        }
    };

    // ---- query inputs first ---------------------------------------------------
    // The vector-memory counter retires loads in issue order: whatever the
    // set-up waits for is issued before the ring prologue, so that wait does
    // not also wait for the KV rows.
    constexpr int kQLoads = LOADS * (LY::kElemsPerLoad / 8);  // 16-B query loads per head
    constexpr int kHeadItems = (GROUP + 1) * (HD / 2);        // per KV head: Q pairs, then K pairs
    constexpr int kRopeItems = KVH * kHeadItems;
    constexpr int RIT = (kRopeItems + kThreads - 1) / kThreads;
    uint16_t rx[RIT], ry[RIT];
    float rc[RIT], rs[RIT];
    uint16_t vnew = 0;
    uint4 qraw[FUSED ? 1 : GROUP][kQLoads];
    if constexpr (FUSED) {
        const int half = HD / 2;
        const uint16_t* qkv = a.q + size_t(b) * a.q_stride;
        const float* crow = a.cos_t + size_t(pos) * half;
        const float* srow = a.sin_t + size_t(pos) * half;
        const int nq = nkv * GROUP;
        // Every thread loads, items past the end and other splits' K items at a
        // clamped, in-bounds index (the rotation below skips them): a load
        // under a branch would need its value moved at the join, and the
        // compiler then waits for it before the ring prologue is issued.
#pragma unroll
        for (int r = 0; r < RIT; ++r) {
            const int it = min(tid + r * kThreads, kRopeItems - 1);
            const int hh = hw * KVH + it / kHeadItems;  // the item's KV head
            const int gh = (it % kHeadItems) / half, d = it % half;
            const uint16_t* src = qkv + size_t(gh < GROUP ? hh * GROUP + gh : nq + hh) * HD;
            rx[r] = src[d];
            ry[r] = src[d + half];
            rc[r] = crow[d];
            rs[r] = srow[d];
        }
        vnew = qkv[size_t(nq + nkv + hw * KVH) * HD + tid % (KVH * HD)];  // used by the owner
    } else {
        const uint16_t* qb = a.q + size_t(b) * a.q_stride + size_t(h) * GROUP * HD;
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh)
#pragma unroll
            for (int i = 0; i < LOADS; ++i)
#pragma unroll
                for (int w = 0; w < LY::kElemsPerLoad / 8; ++w)
                    qraw[gh][i * (LY::kElemsPerLoad / 8) + w] =
                        *reinterpret_cast<const uint4*>(qb + gh * HD + LY::dim(i, j, 0) + w * 8);
    }

    // ---- ring prologue: the first NB row-steps go in flight ----------------
    // (the scheduling barrier keeps the query loads ahead of the KV loads)
    __builtin_amdgcn_sched_barrier(0);
    Row ring[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) load_row(ring[i], min(i, n_steps - 1), kStream);
    AF_STAMP(1);

    // ---- query fragment -----------------------------------------------------
    half2_t qv[GROUP][EPL / 2];
    auto unpack_q = [&](int gh, int slot, const uint4 raw) {
        const int i = slot / (LY::kElemsPerLoad / 8), w = slot % (LY::kElemsPerLoad / 8);
        const int p0 = i * (LY::kElemsPerLoad / 2) + w * 4;
        qv[gh][p0 + 0] = __builtin_bit_cast(half2_t, raw.x);
        qv[gh][p0 + 1] = __builtin_bit_cast(half2_t, raw.y);
        qv[gh][p0 + 2] = __builtin_bit_cast(half2_t, raw.z);
        qv[gh][p0 + 3] = __builtin_bit_cast(half2_t, raw.w);
    };
    if constexpr (FUSED) {
        // RoPE of the GROUP query heads into LDS (every split computes the same
        // bits); the owner also rotates K head h, and stages the new K/V row.
        const int half = HD / 2;
        const int nq = nkv * GROUP;
#pragma unroll
        for (int r = 0; r < RIT; ++r) {
            const int it = tid + r * kThreads;
            const int kv = it / kHeadItems, hh = hw * KVH + kv;
            const int gh = (it % kHeadItems) / half, d = it % half;
            if (it >= kRopeItems || !(gh < GROUP || owner)) continue;
            uint16_t xo, yo;
            rope_rotate(rx[r], ry[r], rc[r], rs[r], xo, yo);
            if (gh < GROUP) {
                s_q[(kv * GROUP + gh) * HD + d] = xo;
                s_q[(kv * GROUP + gh) * HD + d + half] = yo;
            } else {
                uint16_t* kh = a.q + size_t(b) * a.q_stride + size_t(nq + hh) * HD;
                kh[d] = xo;  // K is rotated in place (only this workgroup reads K head hh)
                kh[d + half] = yo;
                if constexpr (FP8) {
                    uint8_t* kn = reinterpret_cast<uint8_t*>(s_new + kv * 2 * V16);
                    kn[d] = uint8_t(quantize_fp8_dev(xo, a.scales[hh]));
                    kn[d + half] = uint8_t(quantize_fp8_dev(yo, a.scales[hh]));
                } else {
                    uint16_t* kn = reinterpret_cast<uint16_t*>(s_new + kv * 2 * V16);
                    kn[d] = xo;
                    kn[d + half] = yo;
                }
            }
        }
        if (owner && tid < KVH * HD) {
            const int kv = tid / HD, e = tid % HD;
            if constexpr (FP8) {
                reinterpret_cast<uint8_t*>(s_new + kv * 2 * V16)[LY::kRowBytes + e] =
                    uint8_t(quantize_fp8_dev(vnew, a.scales[nkv + hw * KVH + kv]));
            } else {
                reinterpret_cast<uint16_t*>(s_new + kv * 2 * V16)[HD + e] = vnew;
            }
        }
        __syncthreads();
        if (owner) {  // append: the K/V rows of the workgroup's heads to the destination row
            const int64_t row = a.slots ? a.slots[b] : int64_t(pos);
            if (tid < KVH * 2 * V16) {
                const int kv = tid / (2 * V16), r = tid % (2 * V16);
                uint8_t* dst = (r < V16 ? a.k : a.v) + row * a.row_bytes +
                               size_t(hw * KVH + kv) * LY::kRowBytes + (r % V16) * 16;
                *reinterpret_cast<uint4*>(dst) = s_new[tid];
            }
        }
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh)
#pragma unroll
            for (int sl = 0; sl < kQLoads; ++sl) {
                const int i = sl / (LY::kElemsPerLoad / 8), w = sl % (LY::kElemsPerLoad / 8);
                unpack_q(gh, sl, *reinterpret_cast<const uint4*>(
                                     &s_q[(sub * GROUP + gh) * HD + LY::dim(i, j, 0) + w * 8]));
            }
    } else {
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh)
#pragma unroll
            for (int sl = 0; sl < kQLoads; ++sl) unpack_q(gh, sl, qraw[gh][sl]);
    }

    float qk_scale = a.qk_scale;
    if constexpr (FP8) qk_scale *= a.scales[h];

    float m_run[GROUP], l_run[GROUP], acc[GROUP][EPL];
#pragma unroll
    for (int gh = 0; gh < GROUP; ++gh) {
        m_run[gh] = kEmptyMax;  // finite: exp2(-inf - kEmptyMax) = 0 for masked rows
        l_run[gh] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[gh][e] = 0.f;
    }

    // Scores of one row-step for the GROUP query heads (log2 units, masked rows
    // -inf); the fused kernel first substitutes the appended row from LDS.
    auto score_row = [&](Row& r, int step, float (&s)[GROUP]) {
        const int t = lane_t0 + step * STEP;
        if constexpr (FUSED) {
            // The new token (and padding past it) takes the appended row from LDS.
            if (t >= L - 1) {
#pragma unroll
                for (int i = 0; i < LOADS; ++i) {
                    r.k[i] = s_new[sub * 2 * V16 + (i * 128 + j * 16) / 16];
                    r.v[i] = s_new[sub * 2 * V16 + V16 + (i * 128 + j * 16) / 16];
                }
            }
        }
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh) s[gh] = 0.f;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t w4[4] = {r.k[i].x, r.k[i].y, r.k[i].z, r.k[i].w};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                if constexpr (FP8) {
                    const half2_t k01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(w4[w]), 1.0f, false);
                    const half2_t k23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(w4[w]), 1.0f, true);
                    const int p = i * 8 + w * 2;
#pragma unroll
                    for (int gh = 0; gh < GROUP; ++gh) {
                        s[gh] = __builtin_amdgcn_fdot2(k01, qv[gh][p], s[gh], false);
                        s[gh] = __builtin_amdgcn_fdot2(k23, qv[gh][p + 1], s[gh], false);
                    }
                } else {
                    const half2_t kk = __builtin_bit_cast(half2_t, w4[w]);
                    const int p = i * 4 + w;
#pragma unroll
                    for (int gh = 0; gh < GROUP; ++gh)
                        s[gh] = __builtin_amdgcn_fdot2(kk, qv[gh][p], s[gh], false);
                }
            }
        }
        const bool valid = t < t_valid;
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh) {
            const float x = group8_sum(s[gh]) * qk_scale;
            s[gh] = valid ? x : -INFINITY;
        }
    };

    auto process_row = [&](Row& r, int step) {
        float s[GROUP];
        score_row(r, step, s);
        // Per-lane running max with a lazy rescale: the reference point only
        // moves when a score exceeds it by more than 2^kLazyLog2, so p <= 2^8
        // and the (rare) accumulator rescale replaces a cross-lane max per row.
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh) {
            if (s[gh] > m_run[gh] + kLazyLog2) {
                const float m_new = s[gh];
                const float alpha = fast_exp2(m_run[gh] - m_new);
                l_run[gh] *= alpha;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[gh][e] *= alpha;
                m_run[gh] = m_new;
            }
        }
        float p[GROUP];
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh) {
            p[gh] = fast_exp2(s[gh] - m_run[gh]);
            l_run[gh] += p[gh];
        }
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t w4[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
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
    };

    // FP8: two row-steps at once. One lazy-max check covers both rows (the
    // reference point still only moves past 2^kLazyLog2, so p <= 2^8), and P.V
    // runs on v_dot2_f32_f16 across the two rows: a byte permute puts dimension
    // e of both rows' V codes side by side, the FP8 -> f16 conversion is exact,
    // and (p0, p1) are rounded to f16 (relative 2^-11). 72 VALU instructions
    // per pair for V where two single rows take 112.
    auto process_pair = [&](Row& r0, int step0, Row& r1, int step1) {
        float s0[GROUP], s1[GROUP];
        score_row(r0, step0, s0);
        __builtin_amdgcn_sched_barrier(0);  // one row's K temporaries live at a time
        score_row(r1, step1, s1);
        __builtin_amdgcn_sched_barrier(0);
        half2_t pp[GROUP];
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh) {
            const float sm = fmaxf(s0[gh], s1[gh]);
            if (sm > m_run[gh] + kLazyLog2) {
                const float alpha = fast_exp2(m_run[gh] - sm);
                l_run[gh] *= alpha;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[gh][e] *= alpha;
                m_run[gh] = sm;
            }
            const float p0 = fast_exp2(s0[gh] - m_run[gh]);
            const float p1 = fast_exp2(s1[gh] - m_run[gh]);
            l_run[gh] += p0 + p1;
            pp[gh] = half2_t{f16(p0), f16(p1)};
        }
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t a4[4] = {r0.v[i].x, r0.v[i].y, r0.v[i].z, r0.v[i].w};
            const uint32_t b4[4] = {r1.v[i].x, r1.v[i].y, r1.v[i].z, r1.v[i].w};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                // bytes (r0.b0, r1.b0, r0.b1, r1.b1) and (r0.b2, r1.b2, r0.b3, r1.b3)
                const uint32_t lo = __builtin_amdgcn_perm(a4[w], b4[w], 0x01050004u);
                const uint32_t hi = __builtin_amdgcn_perm(a4[w], b4[w], 0x03070206u);
                const half2_t d[4] = {__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(lo), 1.0f, false),
                                      __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(lo), 1.0f, true),
                                      __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(hi), 1.0f, false),
                                      __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(hi), 1.0f, true)};
                const int e = i * 16 + w * 4;
#pragma unroll
                for (int gh = 0; gh < GROUP; ++gh)
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        acc[gh][e + u] = __builtin_amdgcn_fdot2(pp[gh], d[u], acc[gh][e + u], false);
            }
        }
    };

    // ---- main loop: a ring of NB row-steps per lane -------------------------
    // Each slot is consumed and refilled with the step NB ahead. Whole rounds
    // keep the loop single-exit with the same load sequence on every path, so
    // the compiler waits only for the slot being consumed; the last partial
    // round is drained without refills. Only the last whole round's refills
    // can reach past the end, where they re-read the split's last step. In
    // paged kernels that round is peeled and loads with the default policy,
    // so the re-reads hit L2 instead of fetching the streamed lines again
    // (configs[4]-size FP8 batches: 3% less time; batch-1 contiguous launches
    // measured 1% slower with it and keep one loop).
    constexpr int kPeel = PAGED ? 1 : 0;
    AF_STAMP(2);
    const int n_full = n_steps / NB;
    if constexpr (FP8) {  // slots consumed and refilled two at a time
        static_assert(NB % 2 == 0, "FP8 ring pairs slots");
        auto round_pairs = [&](int round, auto stream) {
#pragma unroll
            for (int i = 0; i < NB; i += 2) {
                const int step = round * NB + i;
                process_pair(ring[i], step, ring[i + 1], step + 1);
                load_row(ring[i], min(step + NB, n_steps - 1), stream);
                load_row(ring[i + 1], min(step + 1 + NB, n_steps - 1), stream);
            }
        };
        for (int round = 0; round + kPeel < n_full; ++round) round_pairs(round, kStream);
        if (kPeel && n_full > 0) round_pairs(n_full - 1, kDefault);
        const int rem = n_steps - n_full * NB;
#pragma unroll
        for (int i = 0; i < NB; ++i)  // the drain row by row (a paired drain costs ~30 VGPRs)
            if (i < rem) process_row(ring[i], n_full * NB + i);
    } else {
        auto round_rows = [&](int round, auto stream) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int step = round * NB + i;
                process_row(ring[i], step);
                load_row(ring[i], min(step + NB, n_steps - 1), stream);
            }
        };
        for (int round = 0; round + kPeel < n_full; ++round) round_rows(round, kStream);
        if (kPeel && n_full > 0) round_rows(n_full - 1, kDefault);
        const int rem = n_steps - n_full * NB;
#pragma unroll
        for (int i = 0; i < NB; ++i)
            if (i < rem) process_row(ring[i], n_full * NB + i);
    }

    AF_STAMP(3);
    if constexpr (PERSIST)  // the claim issued at the item's start has long returned
        if (tid == 0) s_next = next_item;

    // ---- merge: token groups in registers, then the workgroup in LDS -------
    if constexpr (!PAIR) {
        // Lanes i and i+8 of a 16-lane row hold token groups g, g^1 with the
        // same head-dim slice; one row_ror:8 DPP add merges the pair onto its
        // larger reference. Lanes 0..7 of each row then hold one partial
        // (m, l, o[]) and the kParts = 4 * kWaves partials per head are summed
        // through LDS.
        // One v_mul and one v_add_f32 with the DPP operand per value: no
        // contraction (the DPP operand cannot be an FMA's accumulator), and
        // the adds stay here, with every lane active (sunk into the
        // lanes-0..7 branch below they could not read a disabled lane
        // through DPP and would need a v_mov_dpp each).
#pragma unroll
        for (int gh = 0; gh < GROUP; ++gh) {
#pragma clang fp contract(off)
            const float mp = fmaxf(m_run[gh], dpp<0x128>(m_run[gh]));
            const float f = fast_exp2(m_run[gh] - mp);  // groups that saw no row hold l = acc = 0
            const float l = l_run[gh] * f;
            l_run[gh] = l + dpp<0x128>(l);
            asm volatile("" ::"v"(l_run[gh]));
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const float x = acc[gh][e] * f;
                acc[gh][e] = x + dpp<0x128>(x);
                asm volatile("" ::"v"(acc[gh][e]));
            }
            m_run[gh] = mp;
        }
    } else {
        // The four 16-lane rows hold token groups 0..3 of both heads (lanes
        // 0-7 / 8-15 of each row): merge rows 0+1 and 2+3 (v_permlane16_swap),
        // then the halves (v_permlane32_swap). Every lane ends with the wave's
        // partial for its head and head-dim slice.
        auto merge_rows = [&](auto swap) {
#pragma unroll
            for (int gh = 0; gh < GROUP; ++gh) {
                uint32_t ma = __builtin_bit_cast(uint32_t, m_run[gh]), mb = ma;
                swap(ma, mb);
                const float m0 = __builtin_bit_cast(float, ma), m1 = __builtin_bit_cast(float, mb);
                const float mp = fmaxf(m0, m1);
                const float f0 = fast_exp2(m0 - mp), f1 = fast_exp2(m1 - mp);
                uint32_t la = __builtin_bit_cast(uint32_t, l_run[gh]), lb = la;
                swap(la, lb);
                l_run[gh] = __builtin_bit_cast(float, la) * f0 + __builtin_bit_cast(float, lb) * f1;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    uint32_t xa = __builtin_bit_cast(uint32_t, acc[gh][e]), xb = xa;
                    swap(xa, xb);
                    acc[gh][e] = __builtin_bit_cast(float, xa) * f0 + __builtin_bit_cast(float, xb) * f1;
                }
                m_run[gh] = mp;
            }
        };
        merge_rows([](uint32_t& x, uint32_t& y) { swap16(x, y); });
        merge_rows([](uint32_t& x, uint32_t& y) { swap32(x, y); });
    }
    {
        const int part = PAIR ? wave : wave * 4 + (lane >> 4);
        if (PAIR ? lane < 16 : (lane & 15) < kLanesPerRow) {
#pragma unroll
            for (int gh = 0; gh < GROUP; ++gh) {
                const int qh = sub * GROUP + gh;  // the workgroup's query head
#pragma unroll
                for (int i = 0; i < LOADS; ++i)
#pragma unroll
                    for (int u = 0; u < LY::kElemsPerLoad; u += 4)
                        *reinterpret_cast<float4*>(&s_acc[part][qh * HD + LY::dim(i, j, u)]) =
                            make_float4(acc[gh][i * LY::kElemsPerLoad + u],
                                        acc[gh][i * LY::kElemsPerLoad + u + 1],
                                        acc[gh][i * LY::kElemsPerLoad + u + 2],
                                        acc[gh][i * LY::kElemsPerLoad + u + 3]);
                if (j == 0) {
                    s_pm[part][qh] = m_run[gh];
                    s_pl[part][qh] = l_run[gh];
                }
            }
        }
    }
    __syncthreads();
    AF_STAMP(4);
    if constexpr (PERSIST) {
        // The next item's block-table window (thread t: entry t, up to kThreads
        // entries): loaded here, it arrives while this item merges and
        // publishes, and the next item stages it from registers.
        int nb = 0, first = 0, count = 0;
        if (next_window(s_next, &nb, &first, &count)) {
            const int e = min(tid, count - 1);
            nx_entry = a.tables[size_t(nb) * a.max_blocks + first + e];
        }
    }

    // ---- merge the partials: the output, or this split's partial ------------
    // Thread t owns head-dim pair (2t, 2t+1).
    const size_t rec = (size_t(b) * nhw + hw) * a.rec_stride;  // first record of (b, hw)
    const size_t own = rec + a.pre_records + split;            // this split's record
    for (int q2 = tid; q2 < GHD / 2; q2 += kThreads) {
        const int gh = (2 * q2) / HD;
        // V scale of the KV head that query head gh reads (not this lane's head:
        // with pairs, thread t may merge the other head's output)
        const float v_scale = FP8 ? a.scales[nkv + hw * KVH + gh / GROUP] : 1.0f;
        float M = -INFINITY;
#pragma unroll
        for (int p = 0; p < kParts; ++p) M = fmaxf(M, s_pm[p][gh]);
        float lsum = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (int p = 0; p < kParts; ++p) {
            const float f = fast_exp2(s_pm[p][gh] - M);  // 0 for a partial that saw no token
            lsum += f * s_pl[p][gh];
            const float2 v = *reinterpret_cast<const float2*>(&s_acc[p][2 * q2]);
            o0 += f * v.x;
            o1 += f * v.y;
        }
        if (direct) {
            const uint32_t pair = uint32_t(__builtin_bit_cast(uint16_t, f16(o0 * v_scale / lsum))) |
                                  (uint32_t(__builtin_bit_cast(uint16_t, f16(o1 * v_scale / lsum))) << 16);
            *reinterpret_cast<uint32_t*>(out_b + 2 * q2) = pair;
        } else {  // the partial, as 64-bit agent-scope stores
            const uint64_t v = uint64_t(__builtin_bit_cast(uint32_t, o0 * v_scale)) |
                               (uint64_t(__builtin_bit_cast(uint32_t, o1 * v_scale)) << 32);
            __hip_atomic_store(reinterpret_cast<uint64_t*>(a.part_o + own * GHD) + q2, v,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((2 * q2) % HD == 0) {
                store_agent(a.part_ml + own * 2 * GQ + gh, M);
                store_agent(a.part_ml + own * 2 * GQ + GQ + gh, lsum);
            }
        }
    }
    AF_STAMP(5);
    if (direct) {
        if constexpr (FUSED) {  // the only reader of these Q heads: rotate in place now
            uint16_t* qd = a.q + size_t(b) * a.q_stride + size_t(hw) * GHD;
            for (int o = tid; o < GHD; o += kThreads) qd[o] = s_q[o];
        }
        return;
    }

    // ---- arrival: the last split of (b, h) to finish combines --------------
    // No release/acquire fence: a device-wide fence costs an L2 write-back and
    // invalidate per workgroup, more than the kernel itself. Correctness rests
    // instead on these gfx950 (gfx9-family) rules, which the language-level
    // model does not promise for relaxed atomics:
    //  1. An agent-scope relaxed store lowers to `global_store ... sc1`. The
    //     scope bits make it write through the CU's L1 and this XCD's L2 to the
    //     memory side every XCD reads (MALL / HBM).
    //  2. On gfx9 the vmcnt counter covers stores as well as loads (there is
    //     no separate store counter as on gfx10+), and a store retires from it
    //     only once acknowledged at its scope. So `s_waitcnt vmcnt(0)` below
    //     returns only after this wave's partials are visible device-wide.
    //  3. `s_barrier` after that wait orders the four waves. The counter's
    //     `global_atomic_add` (agent scope, returning) is issued by thread 0
    //     after the barrier, so after every wave's partials are visible.
    //     Device atomics are performed at the memory side, one total order.
    //  4. The last arrival reads partials with agent-scope relaxed loads
    //     (`global_load ... sc1`, served from the memory side, not a stale
    //     L1/L2 line). They sit behind the __syncthreads that publishes
    //     s_last, a workgroup-scope fence no atomic load is hoisted above, and
    //     the hardware issues them in program order after the branch.
    // tests/test_combine_isa.py compiles this file and checks the emitted
    // order of these instructions; af_common.h rejects any other target.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    AF_STAMP(6);
    if constexpr (COMB) {  // the dedicated combiner reads the partial once the flag is set
        if (tid == 0)
            __hip_atomic_store(a.flags + (size_t(b) * nhw + hw) * kCombSplits + split, 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (tid == 0) {
        uint32_t* ctr = a.counters + size_t(b) * nhw + hw;
        const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev == uint32_t(n_active - 1);
        if (last)  // every other split has arrived: re-arm for the next launch
            __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;

    // ---- combine ------------------------------------------------------------
    // Thread t owns output floats 2t, 2t+1 and reads them from CB splits per
    // batch. The (m, l) loads and the first batch are issued before anything
    // waits on them; the split weights are computed while the batch is in
    // flight.
    constexpr int CB = 16;  // splits per batch
    constexpr int MLPT = (2 * GQ * kMaxSplits + kThreads - 1) / kThreads;
    const int n_rec = pre_used + n_active;  // shared-prefix records, then the splits'
    const int n_ml = n_rec * 2 * GQ;
    const size_t rec0 = rec + (a.pre_records - pre_used);  // first record merged
    const float* ml = a.part_ml + rec0 * 2 * GQ;
    const uint64_t* po = reinterpret_cast<const uint64_t*>(a.part_o + rec0 * GHD);
    float mlv[MLPT];
#pragma unroll
    for (int r = 0; r < MLPT; ++r) {
        const int e = tid + r * kThreads;
        mlv[r] = e < n_ml ? load_agent(ml + e) : 0.f;
    }
    uint64_t val[CB];
    auto issue = [&](int q2, int base) {
#pragma unroll
        for (int k = 0; k < CB; ++k)
            val[k] = __hip_atomic_load(po + size_t(min(base + k, n_rec - 1)) * (GHD / 2) + q2,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    issue(min(tid, GHD / 2 - 1), 0);
#pragma unroll
    for (int r = 0; r < MLPT; ++r) {
        const int e = tid + r * kThreads;
        if (e < n_ml) s_ml[e] = mlv[r];
    }
    __syncthreads();
    // split weights w = exp2(m - M) / sum_s exp2(m_s - M) l_s, one wave per head
    // (up to 64 records: lane s holds record s, as in combine_dedicated, so the
    // two merges give the same bits)
    for (int gh = wave; gh < GQ; gh += kWaves) {
        if (n_rec <= 64) {
            const bool has = lane < n_rec;
            const float w = merge_weight(has ? s_ml[lane * 2 * GQ + gh] : -INFINITY,
                                         has ? s_ml[lane * 2 * GQ + GQ + gh] : 0.f);
            if (has) s_wt[gh][lane] = w;
            continue;
        }
        float mx = -INFINITY;
        for (int sp = lane; sp < n_rec; sp += 64) mx = fmaxf(mx, s_ml[sp * 2 * GQ + gh]);
        mx = wave_max(mx);
        float ls = 0.f;
        for (int sp = lane; sp < n_rec; sp += 64)
            ls += fast_exp2(s_ml[sp * 2 * GQ + gh] - mx) * s_ml[sp * 2 * GQ + GQ + gh];
        const float inv = 1.0f / wave_sum(ls);
        for (int sp = lane; sp < n_rec; sp += 64)
            s_wt[gh][sp] = fast_exp2(s_ml[sp * 2 * GQ + gh] - mx) * inv;
    }
    __syncthreads();
    for (int q2 = tid; q2 < GHD / 2; q2 += kThreads) {
        const int gh = (2 * q2) / HD;
        float r0 = 0.f, r1 = 0.f;
        for (int base = 0; base < n_rec; base += CB) {
            if (base > 0 || q2 != tid) issue(q2, base);
#pragma unroll
            for (int k4 = 0; k4 < CB; k4 += 4) {
                const float4 w4 = *reinterpret_cast<const float4*>(&s_wt[gh][base + k4]);
                const float wk[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (base + k4 + u < n_rec) {
                        const uint64_t v = val[k4 + u];
                        r0 = fmaf(wk[u], __builtin_bit_cast(float, uint32_t(v)), r0);
                        r1 = fmaf(wk[u], __builtin_bit_cast(float, uint32_t(v >> 32)), r1);
                    }
                }
            }
        }
        const uint32_t pair = uint32_t(__builtin_bit_cast(uint16_t, f16(r0))) |
                              (uint32_t(__builtin_bit_cast(uint16_t, f16(r1))) << 16);
        *reinterpret_cast<uint32_t*>(out_b + 2 * q2) = pair;
        if constexpr (FUSED)
            *reinterpret_cast<uint32_t*>(a.q + size_t(b) * a.q_stride + size_t(hw) * GHD + 2 * q2) =
                *reinterpret_cast<const uint32_t*>(&s_q[2 * q2]);
    }
    AF_STAMP(10);
}

// One workgroup = (sequence b, KV head h, split), or with PAIR (sequence b,
// KV heads 2hw and 2hw+1, split): then GQ = 2 GROUP query heads share the
// workgroup's records, merge and combine. See the file comment.
template <int HD, int GROUP, bool FP8, bool PAGED, bool FUSED, bool PAIR, bool COMB, bool CACHED>
__device__ __forceinline__ void decode_attn_body(const AttnArgs& a) {
    constexpr int KVH = PAIR ? 2 : 1;          // KV heads per workgroup
    constexpr int GHD = GROUP * KVH * HD;      // output width of the workgroup
    constexpr int STEP = kWaves * (64 / (kLanesPerRow * KVH));  // token rows per workgroup step

    const int tid = threadIdx.x;
    const int nkv = a.n_kv_heads;
    const int nhw = nkv / KVH;  // workgroups per (sequence, split)
    int id = blockIdx.x;
    AF_STAMP_ENTRY();
    // A dedicated combiner decodes as split 0 of its (sequence, KV head).
    const bool comb = COMB && id >= a.split_wgs;
    if (comb) {
        const int c = id - a.split_wgs;
        id = (c / nhw) * a.num_splits * nhw + c % nhw;
    }
    int hw, split, b;
    int Lc = 0;  // compact grid: the length sequence b attends, from the mapping
    if (PAGED && a.compact) {
        // Sequence bb owns nhw * splits(L_bb) consecutive workgroup ids.
        auto length = [&](int bb) {
            if constexpr (FUSED) {  // the length the fused step attends (0: out of range)
                const int pb = a.positions ? a.positions[bb] : a.pos_host;
                const int64_t rb = a.slots ? a.slots[bb] : int64_t(pb);
                const bool ok = pb >= 0 && pb < a.max_pos && pb < a.max_seq_len && rb >= 0 &&
                                rb < a.max_rows;
                return ok ? pb + 1 : 0;
            } else {
                return min(a.seq_lens ? a.seq_lens[bb] : a.seq_len_host, a.max_seq_len);
            }
        };
        // an out-of-range fused append keeps one workgroup (per head) that
        // reports it, as an empty sequence keeps one for its zero output
        int64_t first_b;
        if (a.batch <= 64) {
            // The batch fits one wave's lanes: every wave maps on its own (a
            // wave-wide scan and a ballot; no LDS round trip, no barrier).
            const int lane = tid & 63;
            const int Lb = lane < a.batch ? length(lane) : 0;
            const int n = lane < a.batch ? grid_splits(a, Lb, STEP) : 0;
            const int incl = wave_inclusive_sum(n);
            if (id >= int64_t(__builtin_amdgcn_readlane(incl, 63)) * nhw) return;
            // the first sequence whose splits end past id
            b = __builtin_ctzll(__builtin_amdgcn_ballot_w64(int64_t(incl) * nhw > id));
            first_b = __builtin_amdgcn_readlane(incl - n, b);
            Lc = __builtin_amdgcn_readlane(Lb, b);
        } else {
            __shared__ int32_t s_splits[kThreads];     // splits of each sequence
            __shared__ int32_t s_len[kThreads];        // its length
            __shared__ int64_t s_first[kThreads + 1];  // exclusive prefix: its first split
            if (tid < a.batch) {
                const int Lb = length(tid);
                s_len[tid] = Lb;
                s_splits[tid] = grid_splits(a, Lb, STEP);
            }
            __syncthreads();
            block_exclusive_scan(s_splits, s_first, a.batch);
            if (id >= s_first[a.batch] * nhw) return;
            int lo = 0, hi = a.batch - 1;  // the last sequence whose first split is <= id
            while (lo < hi) {
                const int mid = (lo + hi + 1) / 2;
                if (s_first[mid] * nhw <= id) lo = mid; else hi = mid - 1;
            }
            b = lo;
            first_b = s_first[b];
            Lc = s_len[b];
        }
        const int r = id - int(first_b * nhw);
        hw = r % nhw;
        split = r / nhw;
    } else {
        hw = id % nhw;
        id /= nhw;
        split = id % a.num_splits;
        b = id / a.num_splits;
    }

    int L, pos = 0;
    if constexpr (FUSED) {
        bool in_range;
        if (PAGED && a.compact) {  // the mapping checked the position and the slot
            in_range = Lc > 0;
            pos = Lc - 1;
        } else {
            pos = a.positions ? a.positions[b] : a.pos_host;
            const int64_t row = a.slots ? a.slots[b] : int64_t(pos);
            in_range = !(pos < 0 || pos >= a.max_pos || pos >= a.max_seq_len || row < 0 ||
                         row >= a.max_rows);
        }
        if (!in_range) {
            if (tid == 0 && split == 0 && hw == 0 && !comb && a.d_status)
                *a.d_status = AF_ERR_OUT_OF_RANGE;
            return;  // out-of-range append: nothing is written
        }
        L = pos + 1;
    } else if (PAGED && a.compact) {
        L = Lc;
    } else {
        L = a.seq_lens ? a.seq_lens[b] : a.seq_len_host;
        L = min(L, a.max_seq_len);
    }
    uint16_t* out_b = a.out + size_t(b) * a.out_stride + size_t(hw) * GHD;
    if (L <= 0) {  // empty sequence: defined as a zero output
        if (split == 0 && !comb)
            for (int o = tid; o < GHD; o += kThreads) out_b[o] = 0;
        return;
    }
    // Balanced partition of rows [t_lo, L) in whole workgroup steps
    // (STEP rows): C steps use n = min(num_splits, ceil(C / span)) splits
    // and split s owns steps [s*C/n, (s+1)*C/n). t_lo = row_start, the first row
    // after a shared prefix (0 without one). A sequence exactly as long as the
    // prefix gets one split over its last row with every row masked (an empty
    // partial), so the combine still runs over the prefix records. A sequence
    // shorter than the prefix attends its own rows [0, L) through its table
    // and its combine leaves the prefix records out (they cover rows >= L).
    const bool below_prefix = L < a.row_start;
    const int pre_used = below_prefix ? 0 : a.pre_records;  // prefix records this (b, h) merges
    const int t_lo = below_prefix ? 0 : min(a.row_start, L - 1);
    const int total_steps = (L - t_lo + STEP - 1) / STEP;
    const int n_active = grid_splits(a, L, STEP);
    if (split >= n_active) return;
    const int step_begin = int(int64_t(split) * total_steps / n_active);
    const int step_end = int(int64_t(split + 1) * total_steps / n_active);
    const int t_begin = t_lo + step_begin * STEP;
    const int t_end = min(L, t_lo + step_end * STEP);
    const int t_valid = L == a.row_start ? t_begin : t_end;  // rows below t_valid are scored
    const int n_steps = step_end - step_begin;  // >= 1
    const bool direct = n_active == 1 && pre_used == 0;  // no combine: write the output
    if constexpr (COMB) {
        if (comb) {
            if (!direct) combine_dedicated<HD, GROUP, FUSED>(a, b, hw, n_active, pos);
            return;
        }
    }
    const Seg sg{b, hw, split, n_active, pre_used, L, pos, t_begin, t_end, t_valid, n_steps};
    int32_t unused = 0;
    decode_attn_seg<HD, GROUP, FP8, PAGED, FUSED, PAIR, COMB, CACHED>(a, sg, unused);
}


template <int HD, int GROUP, bool FP8, bool PAGED, bool FUSED, bool PAIR, bool COMB,
          bool CACHED = false>
__global__ __launch_bounds__(kThreads) void decode_attn_kernel(const AttnArgs a) {
    decode_attn_body<HD, GROUP, FP8, PAGED, FUSED, PAIR, COMB, CACHED>(a);
}

// The fused pair form holds the RoPE inputs of two KV heads across the ring
// prologue; asking for three workgroups per CU keeps it at 3 waves per SIMD
// (168 VGPRs, no spills for GROUP <= 4) where it would otherwise take 178.
template <int HD, int GROUP, bool FP8, bool PAGED, bool FUSED, bool PAIR, bool CACHED = false>
__global__ __launch_bounds__(kThreads, 3) void decode_attn_kernel_3wg(const AttnArgs a) {
    decode_attn_body<HD, GROUP, FP8, PAGED, FUSED, PAIR, false, CACHED>(a);
}


// ---- persistent form for batched launches ---------------------------------
// Sequences of the persistent form (their row-step counts are scanned in LDS).
constexpr int kMaxPersistBatch = 256;

// Big items of a group with n row-steps: its steps in whole items of c1 (the
// remainder goes out in small items).
__host__ __device__ inline int big_items(int n, int c1) { return n / c1; }

// Workgroup-uniform values read from LDS, moved to scalar registers.
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t uni64(int64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(uint64_t(x)));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(uint64_t(x) >> 32));
    return int64_t((uint64_t(hi) << 32) | lo);
}


// Batched paged decode as a persistent grid (one launch of as many workgroups
// as the device holds at once) that claims work items from a device counter,
// so workgroups on faster CUs (or favoured within a CU) take more of them and
// all finish within about one small item of each other. Every (sequence, KV
// head group) with n row-steps is cut into big_items(n) = n / C1 items of C1
// steps, then small items of C2 steps over the rest (C2 < C1, both set by the
// host so a group has at most rec_stride items); all big items are handed out
// first, then the small ones, so the last items claimed are short. (Moving a
// quarter of every group into small items cost more in per-item set-up and
// merge than it saved at the end.) An item is a split: its record
// slot is its index within its group and the last of the group's items to
// publish merges them (the arrival counter of the grid form). Workgroup w
// starts on item w; further claims go through item_ctr (item = grid size +
// the counter's value), and each workgroup requests its next item before
// streaming the current one, so the claim's round trip is hidden. The last
// workgroup to run out of items (done_ctr) re-zeroes both counters.
template <int HD, int GROUP, bool FP8, bool FUSED, bool PAIR, bool CACHED = false>
__global__ __launch_bounds__(kThreads, GROUP <= 4 ? 3 : 1) void decode_attn_persistent(const AttnArgs a) {
    constexpr int KVH = PAIR ? 2 : 1;
    constexpr int GHD = GROUP * KVH * HD;
    constexpr int STEP = kWaves * (64 / (kLanesPerRow * KVH));
    __shared__ int32_t s_len[kMaxPersistBatch];
    __shared__ int32_t s_cnt[kMaxPersistBatch];     // big items, then small items, of sequence b
    __shared__ int64_t s_pre[kMaxPersistBatch + 1];  // exclusive prefix of s_cnt
    __shared__ int32_t s_item;
    const int tid = threadIdx.x;
    const int B = a.batch;
    const int nhw = a.n_kv_heads / KVH;
    const int C1 = a.item_big, C2 = a.item_small;
    uint32_t* item_ctr = a.counters + kItemCounter;
    uint32_t* done_ctr = a.counters + kDoneCounter;
    // big-item counts of every sequence, then their prefix
    for (int bb = tid; bb < B; bb += kThreads) {
        int L;
        if constexpr (FUSED) {
            const int pos = a.positions[bb];
            const int64_t row = a.slots[bb];
            const bool ok = pos >= 0 && pos < a.max_pos && pos < a.max_seq_len && row >= 0 &&
                            row < a.max_rows;
            if (!ok && blockIdx.x == 0 && a.d_status) *a.d_status = AF_ERR_OUT_OF_RANGE;
            L = ok ? pos + 1 : 0;  // out-of-range append: nothing is written
        } else {
            L = min(a.seq_lens[bb], a.max_seq_len);
        }
        s_len[bb] = L;
        const int n = L > 0 ? (L + STEP - 1) / STEP : 0;
        s_cnt[bb] = big_items(n, C1);
    }
    __syncthreads();
    block_exclusive_scan(s_cnt, s_pre, B);
    const int64_t T1 = uni64(int64_t(nhw) * s_pre[B]);  // big items in all
    __shared__ int64_t s_pre2[kMaxPersistBatch + 1];    // exclusive prefix of small-item counts
    __shared__ int32_t s_big[kMaxPersistBatch];
    for (int bb = tid; bb < B; bb += kThreads) {
        const int L = s_len[bb];
        const int n = L > 0 ? (L + STEP - 1) / STEP : 0;
        const int nb = big_items(n, C1);
        s_big[bb] = nb;
        s_cnt[bb] = (n - nb * C1 + C2 - 1) / C2;
    }
    __syncthreads();
    block_exclusive_scan(s_cnt, s_pre2, B);
    const int64_t T = T1 + uni64(int64_t(nhw) * s_pre2[B]);
    // Empty sequences (unfused, L <= 0) are defined as a zero output.
    if constexpr (!FUSED) {
        for (int p = blockIdx.x; p < B * nhw; p += gridDim.x) {
            if (s_len[p / nhw] > 0) continue;
            uint16_t* o = a.out + size_t(p / nhw) * a.out_stride + size_t(p % nhw) * GHD;
            for (int e = tid; e < GHD; e += kThreads) o[e] = 0;
        }
    }
    // The item's split descriptor (sequence, group, row range).
    auto make_seg = [&](int64_t item) -> Seg {
        const bool big = item < T1;
        const int64_t* pre = big ? s_pre : s_pre2;
        const int64_t i = big ? item : item - T1;
        // the sequence of item i: the last b with nhw * pre[b] <= i
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) / 2;
            if (int64_t(nhw) * pre[mid] <= i) lo = mid; else hi = mid - 1;
        }
        const int b = uni(lo);
        const int nbig = uni(s_big[b]);
        const int cnt = big ? nbig : uni(s_cnt[b]);
        const int64_t r = i - uni64(int64_t(nhw) * pre[b]);
        const int hw = uni(int(r / cnt));
        const int k = uni(int(r % cnt));  // the item's index among its group's big / small items
        const int L = uni(s_len[b]);
        const int nsmall = uni(s_cnt[b]);
        const int step0 = big ? k * C1 : nbig * C1 + k * C2;
        const int steps = big ? C1 : C2;
        Seg sg;
        sg.b = b;
        sg.hw = hw;
        sg.split = big ? k : nbig + k;
        sg.n_active = nbig + nsmall;
        sg.pre_used = 0;
        sg.L = L;
        sg.pos = L - 1;
        sg.t_begin = step0 * STEP;
        sg.t_end = min(L, (step0 + steps) * STEP);
        sg.t_valid = sg.t_end;
        sg.n_steps = (sg.t_end - sg.t_begin + STEP - 1) / STEP;
        sg.staged = 0;
        return sg;
    };
    // The block-table window of item `it` (false past the last item).
    auto window = [&](uint32_t it, int* nb, int* first, int* count) -> bool {
        if (int64_t(it) >= T) return false;
        const Seg nx = make_seg(it);
        *nb = nx.b;
        *first = nx.t_begin >> a.block_shift;
        *count = ((nx.t_end - 1) >> a.block_shift) - *first + 1;
        return *count <= kThreads;
    };
    // Workgroup w starts on item w without a claim (768 claims at once on one
    // counter serialise at the memory side for microseconds); each further
    // item is claimed at the start of the one before it, whose merge then
    // loads the claimed item's block-table window.
    int64_t item = blockIdx.x;
    int staged = 0;
    int32_t nx_entry = 0;  // thread t: entry t of the next item's block-table window
    while (item < T) {
        uint32_t next = 0;  // the following claim, issued before this item streams
        if (tid == 0)
            next = gridDim.x +
                   __hip_atomic_fetch_add(item_ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        Seg sg = make_seg(item);
        sg.staged = staged;
        decode_attn_seg<HD, GROUP, FP8, true, FUSED, PAIR, false, CACHED, true>(a, sg, nx_entry, next,
                                                                           window);
        if (tid == 0) s_item = int(next);
        __syncthreads();  // the item's LDS (block table, partials) is reused by the next
        item = uni(s_item);
        int nb, first, count;
        staged = window(uint32_t(item), &nb, &first, &count);
    }
    if (tid == 0) {  // out of items: the last workgroup re-arms the counters
        const uint32_t prev = __hip_atomic_fetch_add(done_ctr, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        if (prev == gridDim.x - 1) {
            __hip_atomic_store(item_ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(done_ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}
}  // namespace
}  // namespace af

// ============================================================================
// Host side: dispatch, split heuristics, workspaces, C ABI.
// ============================================================================
namespace af {
namespace {

template <int HD, int GROUP, bool FP8, bool PAGED, bool FUSED, bool PAIR = false, bool COMB = false,
          bool CACHED = false>
int launch_attn(const AttnArgs& a, int grid, hipStream_t s) {
    if constexpr (COMB && (HD != 128 || GROUP > kWaves)) {
        return AF_ERR_UNSUPPORTED;  // the combiner's waves serve one query head each
    } else {
        if constexpr (FUSED && PAIR && GROUP <= 4)
            hipLaunchKernelGGL((decode_attn_kernel_3wg<HD, GROUP, FP8, PAGED, FUSED, PAIR, CACHED>),
                               dim3(grid), dim3(kThreads), 0, s, a);
        else
            hipLaunchKernelGGL((decode_attn_kernel<HD, GROUP, FP8, PAGED, FUSED, PAIR, COMB, CACHED>),
                               dim3(grid), dim3(kThreads), 0, s, a);
        return int(hipGetLastError());
    }
}

template <int HD, bool FP8, bool PAGED, bool FUSED, bool PAIR = false, bool COMB = false,
          bool CACHED = false>
int dispatch_group(const AttnArgs& a, int group, int grid, hipStream_t s) {
    switch (group) {
        case 1: return launch_attn<HD, 1, FP8, PAGED, FUSED, PAIR, COMB, CACHED>(a, grid, s);
        case 2: return launch_attn<HD, 2, FP8, PAGED, FUSED, PAIR, COMB, CACHED>(a, grid, s);
        case 3: return launch_attn<HD, 3, FP8, PAGED, FUSED, PAIR, COMB, CACHED>(a, grid, s);
        case 4: return launch_attn<HD, 4, FP8, PAGED, FUSED, PAIR, COMB, CACHED>(a, grid, s);
        case 8: return launch_attn<HD, 8, FP8, PAGED, FUSED, PAIR, COMB, CACHED>(a, grid, s);
        default: return AF_ERR_UNSUPPORTED;
    }
}

// The fp16 kernels; contiguous launches may take the dedicated-combiner form
// (AttnArgs::split_wgs > 0); paged launches over shared blocks the CACHED form.
template <int HD, bool PAGED, bool FUSED>
int dispatch_fp16(const AttnArgs& a, int group, int grid, hipStream_t s) {
    if constexpr (!PAGED) {
        if (a.split_wgs > 0) return dispatch_group<HD, false, PAGED, FUSED, false, true>(a, group, grid, s);
    } else {
        if (a.cached_rows)
            return dispatch_group<HD, false, PAGED, FUSED, false, false, true>(a, group, grid, s);
    }
    return dispatch_group<HD, false, PAGED, FUSED>(a, group, grid, s);
}

// FP8 launches without shared-prefix records take KV heads in pairs (the
// prefix launch writes records per single KV head).
bool pair_heads(bool fp8, const AttnArgs& a) {
    return fp8 && a.pre_records == 0 && a.n_kv_heads % 2 == 0;
}

template <bool FUSED>
int dispatch_fused(const AttnArgs& a, int head_dim, int group, bool fp8, bool paged, int grid,
                   hipStream_t s) {
    if (fp8) {
        if (!paged || head_dim != 128) return AF_ERR_UNSUPPORTED;
        if (a.cached_rows) {
            if (pair_heads(fp8, a))
                return dispatch_group<128, true, true, FUSED, true, false, true>(a, group, grid / 2, s);
            return dispatch_group<128, true, true, FUSED, false, false, true>(a, group, grid, s);
        }
        if (pair_heads(fp8, a)) return dispatch_group<128, true, true, FUSED, true>(a, group, grid / 2, s);
        return dispatch_group<128, true, true, FUSED>(a, group, grid, s);
    }
    if (head_dim == 128)
        return paged ? dispatch_fp16<128, true, FUSED>(a, group, grid, s)
                     : dispatch_fp16<128, false, FUSED>(a, group, grid, s);
    if (head_dim == 64)
        return paged ? dispatch_fp16<64, true, FUSED>(a, group, grid, s)
                     : dispatch_fp16<64, false, FUSED>(a, group, grid, s);
    return AF_ERR_UNSUPPORTED;
}

int dispatch(const AttnArgs& a, int head_dim, int group, bool fp8, bool paged, bool fused,
             int grid, hipStream_t s) {
    return fused ? dispatch_fused<true>(a, head_dim, group, fp8, paged, grid, s)
                 : dispatch_fused<false>(a, head_dim, group, fp8, paged, grid, s);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Persistent form: rows of a big item (before the cap on items per group) and
// small items per big one.
constexpr int kBigItemRows = 1024;
constexpr int kSmallItems = 8;

// Most items of a group with up to n_max row-steps, big items of c1 steps and
// small ones of c2. The count grows with n while big_items(n) stays the same,
// so the maximum is at n_max or just before big_items steps up.
// (big_items(n) = k for n in [k c1, (k + 1) c1).)
int max_items(int n_max, int c1, int c2) {
    auto items = [&](int n) {
        const int nb = big_items(n, c1);
        return nb + ceil_div(n - nb * c1, c2);
    };
    int worst = items(n_max);
    for (int k = 1;; ++k) {
        const int n = c1 * k - 1;  // the last n with big_items(n) = k - 1
        if (n > n_max) break;
        if (n >= 1) worst = std::max(worst, items(n));
    }
    return worst;
}

// Item sizes of the persistent form: big items of c1_min steps and small ones
// of c1 / kSmallItems, the small ones coarsened first (up to c1 / 2), then
// both, until every group fits `records` items.
bool plan_items(int n_max, int records, int c1_min, int* c1, int* c2) {
    int a = std::max(1, c1_min), b = std::max(1, a / kSmallItems);
    for (int guard = 0; guard < 64; ++guard) {
        if (max_items(n_max, a, b) <= records) {
            *c1 = a;
            *c2 = b;
            return true;
        }
        if (2 * b <= a / 2) {
            b *= 2;
        } else {
            a *= 2;
            b = std::max(b, a / kSmallItems);
        }
        if (a > n_max + 1 && b > n_max + 1) break;
    }
    return false;
}

// Workgroups of a persistent launch: as many as the device holds at once
// (occupancy x CUs), looked up once per device for each kernel.
template <int HD, int GROUP, bool FP8, bool FUSED, bool PAIR, bool CACHED>
int persistent_grid() {
    static std::mutex mu;
    static std::vector<int> grid;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(mu);
    if (int(grid.size()) <= dev) grid.resize(size_t(dev) + 1, 0);
    if (!grid[size_t(dev)]) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu,
                reinterpret_cast<const void*>(&decode_attn_persistent<HD, GROUP, FP8, FUSED, PAIR, CACHED>),
                kThreads, 0) != hipSuccess)
            return 0;
        grid[size_t(dev)] = std::max(1, per_cu) * device_compute_units();
    }
    return grid[size_t(dev)];
}

template <int HD, int GROUP, bool FP8, bool FUSED, bool PAIR, bool CACHED>
int launch_persistent(const AttnArgs& a, int grid, hipStream_t s) {
    hipLaunchKernelGGL((decode_attn_persistent<HD, GROUP, FP8, FUSED, PAIR, CACHED>), dim3(grid),
                       dim3(kThreads), 0, s, a);
    return int(hipGetLastError());
}

// The persistent form's kernel for (head_dim, group, dtype, fused): `grid` = 0
// returns its grid size; otherwise launches it over `grid` workgroups.
template <bool FP8, bool FUSED, bool PAIR, bool CACHED>
int persistent_group(const AttnArgs& a, int group, int grid, hipStream_t s) {
#define AF_PERSIST_CASE(G)                                                             \
    case G:                                                                            \
        return grid ? launch_persistent<128, G, FP8, FUSED, PAIR, CACHED>(a, grid, s)  \
                    : persistent_grid<128, G, FP8, FUSED, PAIR, CACHED>();
    switch (group) {
        AF_PERSIST_CASE(1)
        AF_PERSIST_CASE(2)
        AF_PERSIST_CASE(3)
        AF_PERSIST_CASE(4)
        AF_PERSIST_CASE(8)
        default: return grid ? AF_ERR_UNSUPPORTED : 0;
    }
#undef AF_PERSIST_CASE
}

template <bool CACHED>
int persistent_dispatch_policy(const AttnArgs& a, int group, bool fp8, bool fused, int grid,
                               hipStream_t s) {
    const bool pair = pair_heads(fp8, a);
    if (fp8) {
        if (pair) return fused ? persistent_group<true, true, true, CACHED>(a, group, grid, s)
                               : persistent_group<true, false, true, CACHED>(a, group, grid, s);
        return fused ? persistent_group<true, true, false, CACHED>(a, group, grid, s)
                     : persistent_group<true, false, false, CACHED>(a, group, grid, s);
    }
    return fused ? persistent_group<false, true, false, CACHED>(a, group, grid, s)
                 : persistent_group<false, false, false, CACHED>(a, group, grid, s);
}

int persistent_dispatch(const AttnArgs& a, int group, bool fp8, bool fused, int grid, hipStream_t s) {
    return a.cached_rows ? persistent_dispatch_policy<true>(a, group, fp8, fused, grid, s)
                         : persistent_dispatch_policy<false>(a, group, fp8, fused, grid, s);
}

// Launches whose split-K tail goes through dedicated combiners instead of the
// last-arriving split: few (sequence, KV head) pairs (combiners are one
// workgroup each, dispatched after every split), at most kCombSplits splits,
// and one output pair per combiner thread.
bool combiner_shape(int group, int head_dim) { return head_dim == 128 && group <= kWaves; }

bool use_combiner(int batch, int n_kv_heads, int num_splits, int group, int head_dim) {
    return num_splits >= 2 && num_splits <= kCombSplits && combiner_shape(group, head_dim) &&
           int64_t(batch) * n_kv_heads <= kCombMaxGroups;
}

float qk_scale_for(int head_dim) { return float(1.4426950408889634 / std::sqrt(double(head_dim))); }

// Zero arrival counters and ready flags (the state each launch leaves behind).
int init_workspace(void* ws, size_t bytes, hipStream_t stream) {
    (void)bytes;
    return fill_u32(ws, 0u, kCounterBytes / 4, stream);
}

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
        int st = init_workspace(p, need, stream);
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

// Batches with at least half a (sequence, KV head) pair per CU balance the work
// per workgroup: every split covers about kBatchSpan tokens, so a sequence's
// split count follows its length. Smaller launches split every sequence the
// same way to fill the CUs.
int default_span(int batch, int n_kv_heads) {
    return int64_t(batch) * n_kv_heads * 2 >= device_compute_units() ? kBatchSpan : kMinSpan;
}

int default_splits_for(int max_seq_len, int batch, int n_kv_heads, bool combiner) {
    if (max_seq_len <= 0) return 1;
    if (default_span(batch, n_kv_heads) == kBatchSpan)
        return std::min(std::max(ceil_div(max_seq_len, kBatchSpan), 1), kMaxSplits);
    const int pairs = std::max(1, batch * n_kv_heads);
    // About 3/4 of a workgroup per CU: measured best on MI355X for batch 1
    // (the split-K combine grows with the split count faster than more
    // workgroups add bandwidth).
    const int cus = device_compute_units();
    const int base = std::max(1, (3 * cus) / (4 * pairs));
    // Long sequences: spans of about 1024 rows, but never more workgroups than
    // CUs. A grid just past the CU count doubles up a few CUs, and the launch
    // then waits on them (ctx 32k on MI355X: 33 splits x 8 heads = 264
    // workgroups ran 40.5 us, 32 splits 29.6 us, 64 splits 31.3 us). A launch
    // that takes the dedicated combiner gives each pair a combiner workgroup,
    // and one more CU per pair left free measured best (ctx 32k, 8 heads: 30 /
    // 31 / 32 splits 28.5 / 28.9 / 29.3 us); the room for splits is then
    // (CUs - 2 pairs) / pairs.
    auto pick = [&](int room) {
        int sp = std::max(base, std::min(ceil_div(max_seq_len, 1024), std::max(1, room)));
        sp = std::min(sp, std::max(1, ceil_div(max_seq_len, kMinSpan)));
        return std::min(std::max(sp, 1), kMaxSplits);
    };
    if (combiner && pairs <= kCombMaxGroups) {
        const int sp = pick((cus - 2 * pairs) / pairs);
        if (sp <= kCombSplits) return sp;  // the launch does take the combiner
    }
    return pick(cus / pairs);
}

int default_splits(int max_seq_len, int batch, int n_kv_heads) {
    return default_splits_for(max_seq_len, batch, n_kv_heads, true);
}

// Smallest split count whose span fits the LDS-staged block table.
static int min_splits_for_table(int max_seq_len, int block_size) {
    const int max_span = (kMaxTableLds - 2) * block_size - 2 * kStepTokens;
    return ceil_div(max_seq_len, max_span);
}

}  // namespace af

using namespace af;

#ifdef AF_PHASE_STAMPS
// Measurement build only: the phase table of the last launch per workgroup
// (uint64 [2048][8], s_memrealtime ticks of 10 ns; 0 = phase not reached).
extern "C" int af_dbg_phase_stamps(void* host, size_t bytes) {
    if (bytes > sizeof(g_phase_stamps)) bytes = sizeof(g_phase_stamps);
    return int(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_phase_stamps), bytes));
}
extern "C" int af_dbg_phase_stamps_clear(void) {
    static uint64_t zeros[kStampWgs][kStampPhases];
    return int(hipMemcpyToSymbol(HIP_SYMBOL(g_phase_stamps), zeros, sizeof(zeros)));
}
#endif

extern "C" size_t af_attention_workspace_size(int batch, int n_q_heads, int n_kv_heads,
                                              int head_dim, int num_splits) {
    if (batch <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0) return 0;
    if (num_splits <= 0 || num_splits > kMaxSplits) num_splits = kMaxSplits;
    return attn_workspace_bytes(batch, n_q_heads, head_dim, num_splits);
}

extern "C" int af_attention_workspace_init(void* workspace, size_t workspace_bytes,
                                           af_stream_t stream) {
    if (!workspace || workspace_bytes < kCounterBytes) return AF_ERR_WORKSPACE;
    return init_workspace(workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int af_attention_default_splits(int max_seq_len, int batch, int n_kv_heads) {
    return default_splits(max_seq_len, batch, n_kv_heads);
}

static int check_heads(int head_dim, int n_q_heads, int n_kv_heads) {
    if (head_dim <= 0 || n_q_heads <= 0 || n_kv_heads <= 0) return AF_ERR_INVALID_ARG;
    if (n_q_heads % n_kv_heads) return AF_ERR_UNSUPPORTED;
    return AF_OK;
}

static int contiguous_attention(void* q, int q_stride, void* k_cache, void* v_cache, void* out,
                                int seq_len, const int32_t* d_seq_len, int max_seq_len,
                                int head_dim, int n_q_heads, int n_kv_heads, int num_splits,
                                void* workspace, size_t workspace_bytes, bool fused,
                                const float* cos_table, const float* sin_table, int pos,
                                const int32_t* d_pos, int32_t* d_status, hipStream_t stream) {
    if (!q || !k_cache || !v_cache || !out || max_seq_len <= 0) return AF_ERR_INVALID_ARG;
    if (int st = check_heads(head_dim, n_q_heads, n_kv_heads)) return st;
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache)) return AF_ERR_INVALID_ARG;
    if (num_splits <= 0)
        num_splits = default_splits_for(max_seq_len, 1, n_kv_heads,
                                        combiner_shape(n_q_heads / n_kv_heads, head_dim));
    if (num_splits > kMaxSplits) return AF_ERR_INVALID_ARG;
    if (n_kv_heads > kMaxCounters) return AF_ERR_UNSUPPORTED;
    if (!workspace || workspace_bytes < attn_workspace_bytes(1, n_q_heads, head_dim, num_splits))
        return AF_ERR_WORKSPACE;
    const AttnWorkspace w = attn_workspace_carve(workspace, 1, n_q_heads, num_splits);
    AttnArgs a{};
    a.q = static_cast<uint16_t*>(q);
    a.q_stride = q_stride;
    a.k = static_cast<uint8_t*>(k_cache);
    a.v = static_cast<uint8_t*>(v_cache);
    a.row_bytes = int64_t(n_kv_heads) * head_dim * 2;
    a.seq_lens = d_seq_len;
    a.seq_len_host = seq_len;
    a.max_seq_len = max_seq_len;
    if (fused) {
        a.positions = d_pos;
        a.pos_host = pos;
        a.max_rows = max_seq_len;
        a.cos_t = cos_table;
        a.sin_t = sin_table;
        a.max_pos = max_seq_len;  // the table covers every cache row
        a.d_status = d_status;
    }
    a.out = static_cast<uint16_t*>(out);
    a.out_stride = int64_t(n_q_heads) * head_dim;
    a.n_kv_heads = n_kv_heads;
    a.num_splits = num_splits;
    a.span_tokens = kMinSpan;
    a.qk_scale = qk_scale_for(head_dim);
    a.part_o = w.part_o;
    a.part_ml = w.part_ml;
    a.counters = w.counters;
    a.rec_stride = num_splits;
    int grid = num_splits * n_kv_heads;
    if (use_combiner(1, n_kv_heads, num_splits, n_q_heads / n_kv_heads, head_dim)) {
        a.flags = w.flags;
        a.split_wgs = grid;
        grid += n_kv_heads;  // one combiner per KV head, dispatched after every split
    }
    return dispatch(a, head_dim, n_q_heads / n_kv_heads, false, false, fused, grid, stream);
}

extern "C" int af_cached_attention_ex(const void* q, const void* k_cache, const void* v_cache,
                                      void* out, int seq_len, const int32_t* d_seq_len,
                                      int max_seq_len, int head_dim, int n_q_heads, int n_kv_heads,
                                      int num_splits, void* workspace, size_t workspace_bytes,
                                      af_stream_t stream) {
    if (!d_seq_len && (seq_len < 0 || seq_len > max_seq_len)) return AF_ERR_OUT_OF_RANGE;
    return contiguous_attention(const_cast<void*>(q), n_q_heads * head_dim,
                                const_cast<void*>(k_cache), const_cast<void*>(v_cache), out,
                                seq_len, d_seq_len, max_seq_len, head_dim, n_q_heads, n_kv_heads,
                                num_splits, workspace, workspace_bytes, false, nullptr, nullptr, 0,
                                nullptr, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int af_decode_attention_fused(void* qkv_out, void* k_cache, void* v_cache,
                                         const float* cos_table, const float* sin_table, int pos,
                                         const int32_t* d_pos, int max_seq, void* out,
                                         int n_q_heads, int n_kv_heads, int head_dim,
                                         int num_splits, void* workspace, size_t workspace_bytes,
                                         int32_t* d_status, af_stream_t stream) {
    if (!cos_table || !sin_table || !aligned16(cos_table) || !aligned16(sin_table))
        return AF_ERR_INVALID_ARG;
    if (!d_pos && (pos < 0 || pos >= max_seq)) return AF_ERR_OUT_OF_RANGE;
    return contiguous_attention(qkv_out, (n_q_heads + 2 * n_kv_heads) * head_dim, k_cache,
                                v_cache, out, 0, nullptr, max_seq, head_dim, n_q_heads, n_kv_heads,
                                num_splits, workspace, workspace_bytes, true, cos_table, sin_table,
                                pos, d_pos, d_status, static_cast<hipStream_t>(stream));
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
                                  n_q_heads, n_kv_heads,
                                  default_splits_for(seq_len, 1, n_kv_heads,
                                                     combiner_shape(n_q_heads / n_kv_heads, head_dim)),
                                  ws,
                                  bytes, stream);
}

// ---- allocation-free form of af_cached_attention ---------------------------
// The split-K workspace of af_cached_attention_noalloc lives in this
// file-scope device array (kScratchBytes per device, held until the process
// ends). Host code never passes the array's name to a kernel: the device
// address comes from hipGetSymbolAddress, once per device, and is kept per
// device in g_scratch_ptr.
constexpr size_t kScratchBytes = size_t(4) * 1024 * 1024 + size_t(128) * 1024;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
static std::mutex g_scratch_mu;
static std::vector<void*> g_scratch_ptr;

// Device address of this device's scratch. The first call on a device looks
// the address up and clears the arrival counters with the fill kernel (stream-
// ordered before the attention launch that follows; every launch leaves its
// counters at zero again). No allocation.
static int scratch_for_device(hipStream_t stream, void** out) {
    int dev = 0;
    AF_TRY_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (int(g_scratch_ptr.size()) <= dev) g_scratch_ptr.resize(size_t(dev) + 1, nullptr);
    if (!g_scratch_ptr[size_t(dev)]) {
        void* p = nullptr;
        AF_TRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return AF_ERR_WORKSPACE;
        if (int st = fill_u32(p, 0u, kCounterBytes / 4, stream)) return st;
        g_scratch_ptr[size_t(dev)] = p;
    }
    *out = g_scratch_ptr[size_t(dev)];
    return AF_OK;
}

extern "C" size_t af_cached_attention_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int af_cached_attention_noalloc(const void* q, const void* k_cache,
                                           const void* v_cache, void* out, int seq_len,
                                           int head_dim, int n_q_heads, int n_kv_heads,
                                           af_stream_t stream) {
    if (seq_len <= 0) return AF_ERR_INVALID_ARG;
    if (int st = check_heads(head_dim, n_q_heads, n_kv_heads)) return st;
    const int splits = default_splits_for(seq_len, 1, n_kv_heads,
                                          combiner_shape(n_q_heads / n_kv_heads, head_dim));
    const size_t need = attn_workspace_bytes(1, n_q_heads, head_dim, splits);
    if (need > kScratchBytes) return AF_ERR_WORKSPACE;  // shape beyond the static scratch
    void* ws = nullptr;
    if (int st = scratch_for_device(static_cast<hipStream_t>(stream), &ws)) return st;
    return af_cached_attention_ex(q, k_cache, v_cache, out, seq_len, nullptr, seq_len, head_dim,
                                  n_q_heads, n_kv_heads, splits, ws, kScratchBytes, stream);
}

// Rows [0, len) shared by every sequence of a launch, mapped by `table`.
struct SharedPrefix {
    const int32_t* table = nullptr;
    int len = 0;
    int splits = 0;  // key splits of the prefix launch; 0 = default
};

// Default key splits of the shared-prefix launch: about one workgroup per CU,
// at least one 64-key tile per split.
static int default_prefix_splits(int prefix_len, int batch, int group, int n_kv_heads) {
    const int per_split = std::max(1, prefix_partial_tiles(batch, group, n_kv_heads));
    int s = std::max(1, device_compute_units() / per_split);
    return std::min(std::min(s, 32), ceil_div(prefix_len, 64));
}

static int paged_attention(void* q, int q_stride, const af_kv_pool* pool, int layer,
                           const int32_t* d_block_tables, int max_blocks_per_seq,
                           const int32_t* d_seq_lens, int batch, int max_seq_len, void* out,
                           int out_stride, int n_q_heads, int num_splits, void* workspace,
                           size_t workspace_bytes, bool fused, const int64_t* d_slots,
                           const int32_t* d_positions, const float* cos_table,
                           const float* sin_table, int max_pos, hipStream_t stream,
                           const SharedPrefix& prefix = SharedPrefix()) {
    if (!q || !pool || !pool->base || !d_block_tables || !out || batch < 0 || max_seq_len < 0 ||
        max_blocks_per_seq <= 0)
        return AF_ERR_INVALID_ARG;
    if (fused ? (!d_slots || !d_positions || !cos_table || !sin_table || max_pos <= 0 ||
                 !aligned16(cos_table) || !aligned16(sin_table))
              : !d_seq_lens)
        return AF_ERR_INVALID_ARG;
    if (layer < 0 || layer >= pool->n_layers || pool->total_blocks <= 0) return AF_ERR_INVALID_ARG;
    if (pool->flags & ~AF_KV_POOL_SHARED_BLOCKS) return AF_ERR_INVALID_ARG;
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
    if (prefix.len < 0 || prefix.splits < 0) return AF_ERR_INVALID_ARG;
    if (prefix.len > 0) {
        if (!prefix.table) return AF_ERR_INVALID_ARG;
        if (hd != 128) return AF_ERR_UNSUPPORTED;
        if (int64_t(max_blocks_per_seq) * bs < prefix.len) return AF_ERR_OUT_OF_RANGE;
        if (prefix.splits > ceil_div(prefix.len, 64)) return AF_ERR_INVALID_ARG;
    }
    if (batch == 0) return AF_OK;
    if (int64_t(batch) * nkv > kMaxCounters) return AF_ERR_UNSUPPORTED;
    // The splits cover the rows after the prefix (at least one row each), or
    // all rows [0, L) of a sequence shorter than the prefix: each split's
    // block-table window must fit the LDS copy for either.
    const int suffix_max = std::max(max_seq_len - prefix.len, 1);
    const int min_sp = min_splits_for_table(std::max(suffix_max, std::min(prefix.len, max_seq_len)), bs);
    int span = kMinSpan;
    bool persistent_ok = false;  // the default partition of a batch may run persistent
    if (num_splits <= 0) {
        num_splits = std::max(default_splits_for(suffix_max, batch, nkv, false), min_sp);
        span = default_span(batch, nkv);
        // (FP8 pools; the fp16 kernel streams faster than its per-item
        // set-up and merge let a persistent workgroup overlap, so fp16 batches
        // keep the grid form)
        persistent_ok = fp8 && span == kBatchSpan && prefix.len == 0 && hd == 128 &&
                        batch <= kMaxPersistBatch;
        if (prefix.len > 0 && span == kBatchSpan) {
            // Batched suffixes behind a shared prefix are short: splits of up to
            // ~256 rows (measured best on MI355X for 64 forks of a 2048-row
            // prefix, suffixes 1..1024), each sequence using as many as its
            // steps allow.
            num_splits = std::max(std::min(ceil_div(suffix_max, 256), kMaxSplits / 2), min_sp);
            span = kMinSpan;
        }
    } else if (num_splits < min_sp) {
        return AF_ERR_INVALID_ARG;
    }
    if (num_splits > kMaxSplits) return AF_ERR_OUT_OF_RANGE;
    int pre = 0;  // prefix records per (sequence, KV head)
    if (prefix.len > 0) {
        pre = prefix.splits;
        if (pre == 0)
            pre = std::max(1, std::min(default_prefix_splits(prefix.len, batch, n_q_heads / nkv, nkv),
                                       kMaxSplits - num_splits));
        if (num_splits + pre > kMaxSplits) return AF_ERR_OUT_OF_RANGE;
    }
    const int rec_stride = num_splits + pre;
    if (!workspace || workspace_bytes < attn_workspace_bytes(batch, n_q_heads, hd, rec_stride))
        return AF_ERR_WORKSPACE;
    const AttnWorkspace w = attn_workspace_carve(workspace, batch, n_q_heads, rec_stride);
    const size_t esz = fp8 ? 1 : 2;
    const size_t slab = size_t(pool->total_blocks) * bs * nkv * hd * esz;
    uint8_t* base = static_cast<uint8_t*>(pool->base);
    AttnArgs a{};
    a.q = static_cast<uint16_t*>(q);
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
    if (fused) {
        a.positions = d_positions;
        a.slots = d_slots;
        a.max_rows = int64_t(pool->total_blocks) * bs;
        a.cos_t = cos_table;
        a.sin_t = sin_table;
        a.max_pos = max_pos;
    }
    a.out = static_cast<uint16_t*>(out);
    a.out_stride = out_stride;
    a.n_kv_heads = nkv;
    a.num_splits = num_splits;
    a.span_tokens = span;
    a.qk_scale = qk_scale_for(hd);
    a.scales = fp8 ? pool->scales + size_t(layer) * 2 * nkv : nullptr;
    a.part_o = w.part_o;
    a.part_ml = w.part_ml;
    a.counters = w.counters;
    a.row_start = prefix.len;
    a.pre_records = pre;
    a.rec_stride = rec_stride;
    a.batch = batch;
    a.cached_rows = (pool->flags & AF_KV_POOL_SHARED_BLOCKS) ? 1 : 0;
    // (Only batched launches without a shared prefix: the shared-prefix form's
    // short suffix splits measured slower with the length scan, configs[3]
    // 55.2 against 51.9 us.)
    a.compact = span == kBatchSpan && pre == 0 && batch <= kThreads;
    const int64_t grid = int64_t(batch) * num_splits * nkv;
    if (grid > INT32_MAX) return AF_ERR_UNSUPPORTED;
    if (pre > 0) {  // the prefix's partials first: records 0 .. pre-1
        PrefixPartialArgs pp{};
        pp.q = a.q;
        pp.q_stride = q_stride;
        pp.k = a.k;
        pp.v = a.v;
        pp.row_bytes = a.row_bytes;
        pp.scales = a.scales;
        pp.table = prefix.table;
        pp.bs_log2 = a.block_shift;
        pp.total_blocks = a.total_blocks;
        pp.prefix_len = prefix.len;
        pp.batch = batch;
        pp.n_kv_heads = nkv;
        pp.group = n_q_heads / nkv;
        pp.key_splits = pre;
        pp.rec_stride = rec_stride;
        pp.part_o = w.part_o;
        pp.part_ml = w.part_ml;
        if (fused) {  // the decode launch ropes Q in place afterwards: rotate a copy here
            pp.cos_t = cos_table;
            pp.sin_t = sin_table;
            pp.positions = d_positions;
            pp.max_pos = max_pos;
        }
        if (int st = launch_prefix_partials(pp, stream)) return st;
    }
    if (persistent_ok) {
        // head_dim 128 batches without a shared prefix, default split count: the
        // persistent form, with item sizes that keep every group within
        // rec_stride items.
        const int group = n_q_heads / nkv;
        const int pgrid = persistent_dispatch(a, group, fp8, fused, 0, stream);
        const int kvh = pair_heads(fp8, a) ? 2 : 1;
        const int step = kWaves * (64 / (kLanesPerRow * kvh));
        int c1 = 0, c2 = 0;
        if (pgrid > 0 && plan_items(ceil_div(max_seq_len, step), rec_stride, kBigItemRows / step,
                                    &c1, &c2) &&
            (c1 * step) / bs + 2 <= kMaxTableLds) {
            a.item_big = c1;
            a.item_small = c2;
            return persistent_dispatch(a, group, fp8, fused, pgrid, stream);
        }
    }
    return dispatch(a, hd, n_q_heads / nkv, fp8, true, fused, int(grid), stream);
}

extern "C" int af_paged_attention(const void* q, int q_stride, const af_kv_pool* pool, int layer,
                                  const int32_t* d_block_tables, int max_blocks_per_seq,
                                  const int32_t* d_seq_lens, int batch, int max_seq_len, void* out,
                                  int out_stride, int n_q_heads, int num_splits, void* workspace,
                                  size_t workspace_bytes, af_stream_t stream) {
    return paged_attention(const_cast<void*>(q), q_stride, pool, layer, d_block_tables,
                           max_blocks_per_seq, d_seq_lens, batch, max_seq_len, out, out_stride,
                           n_q_heads, num_splits, workspace, workspace_bytes, false, nullptr,
                           nullptr, nullptr, nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" int af_paged_decode_fused(void* qkv_out, int batch, const af_kv_pool* pool, int layer,
                                     const int64_t* d_slots, const int32_t* d_positions,
                                     const float* cos_table, const float* sin_table, int max_pos,
                                     const int32_t* d_block_tables, int max_blocks_per_seq,
                                     int max_seq_len, void* out, int out_stride, int n_q_heads,
                                     int num_splits, void* workspace, size_t workspace_bytes,
                                     af_stream_t stream) {
    if (!pool) return AF_ERR_INVALID_ARG;
    const int qkv_stride = (n_q_heads + 2 * pool->n_kv_heads) * pool->head_dim;
    return paged_attention(qkv_out, qkv_stride, pool, layer, d_block_tables, max_blocks_per_seq,
                           nullptr, batch, max_seq_len, out, out_stride, n_q_heads, num_splits,
                           workspace, workspace_bytes, true, d_slots, d_positions, cos_table,
                           sin_table, max_pos, static_cast<hipStream_t>(stream));
}

extern "C" int af_paged_attention_shared_prefix(
    const void* q, int q_stride, const af_kv_pool* pool, int layer, const int32_t* d_prefix_table,
    int prefix_len, int prefix_splits, const int32_t* d_block_tables, int max_blocks_per_seq,
    const int32_t* d_seq_lens, int batch, int max_seq_len, void* out, int out_stride,
    int n_q_heads, int num_splits, void* workspace, size_t workspace_bytes, af_stream_t stream) {
    SharedPrefix sp;
    sp.table = d_prefix_table;
    sp.len = prefix_len;
    sp.splits = prefix_splits;
    return paged_attention(const_cast<void*>(q), q_stride, pool, layer, d_block_tables,
                           max_blocks_per_seq, d_seq_lens, batch, max_seq_len, out, out_stride,
                           n_q_heads, num_splits, workspace, workspace_bytes, false, nullptr,
                           nullptr, nullptr, nullptr, 0, static_cast<hipStream_t>(stream), sp);
}

extern "C" int af_paged_decode_fused_shared_prefix(
    void* qkv_out, int batch, const af_kv_pool* pool, int layer, const int64_t* d_slots,
    const int32_t* d_positions, const float* cos_table, const float* sin_table, int max_pos,
    const int32_t* d_prefix_table, int prefix_len, int prefix_splits,
    const int32_t* d_block_tables, int max_blocks_per_seq, int max_seq_len, void* out,
    int out_stride, int n_q_heads, int num_splits, void* workspace, size_t workspace_bytes,
    af_stream_t stream) {
    if (!pool) return AF_ERR_INVALID_ARG;
    SharedPrefix sp;
    sp.table = d_prefix_table;
    sp.len = prefix_len;
    sp.splits = prefix_splits;
    const int qkv_stride = (n_q_heads + 2 * pool->n_kv_heads) * pool->head_dim;
    return paged_attention(qkv_out, qkv_stride, pool, layer, d_block_tables, max_blocks_per_seq,
                           nullptr, batch, max_seq_len, out, out_stride, n_q_heads, num_splits,
                           workspace, workspace_bytes, true, d_slots, d_positions, cos_table,
                           sin_table, max_pos, static_cast<hipStream_t>(stream), sp);
}
