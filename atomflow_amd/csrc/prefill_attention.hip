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
// Design: a workgroup is 4 waves of one Q head; each wave owns a block of 32
// queries (128 queries per workgroup, two workgroups per CU, so each SIMD has a
// second wave to issue matrix work during the other's softmax).
//  * S^T = K Q^T on v_mfma_f32_32x32x16_f16: the A operand is a K fragment read
//    from LDS, the B operand the query block held in registers for the whole
//    launch (LDS delivers about 64 B/clk per CU, one 1 KB fragment per 16 clk;
//    an MFMA takes 32).
//  * Each lane owns 16 of the 32 scores of one query (lane l^32 the other 16):
//    the softmax is in-lane work plus one v_permlane32_swap.
//  * O^T += V^T P^T. P^T is the S^T accumulator rounded to fp16: within each
//    16-key step the keys are numbered with bits 2 and 3 swapped, which makes the
//    accumulator's register order the operand's k order. V stays row-major in LDS
//    and the V^T operand is read with ds_read_b64_tr_b16 (a 16-lane group reads
//    a 4-key x 16-d block and gets it transposed: lane l, element t = key t,
//    d = l%16), two per operand.
//  * K and V tiles of 64 keys are double-buffered in LDS, XOR-swizzled in 16-byte
//    chunks (K by row%16 for the b128 operand reads, V by 4*(row%4) for the
//    transposing reads). They go from global memory straight into LDS
//    (global_load_lds_dwordx4, no registers); the next tile's loads are issued
//    before the current tile's matrix work: one barrier per tile.
//  * Softmax is online in the log2 domain with lazy rescaling: the running max
//    moves only when a tile's probabilities sum past 2^8 in some lane, so most
//    tiles skip both the tile max and the O^T rescale. The row sum is taken over
//    the fp16 probabilities the P.V product uses.
//  * Paged pools (PAGED): tile rows map through the sequence's block table; the
//    entries for tile kt+1 are fetched during tile kt-1. FP8 pools (FP8) stage
//    tiles through registers and convert E4M3 -> fp16 exactly on the way into
//    LDS; the K scale joins the score scale and the V scale the output.
//  * Workgroups are ordered KV head fastest (consecutive workgroups alternate
//    XCDs, so each XCD's L2 serves one KV head when n_kv_heads divides 8), then
//    Q head, then query tile heaviest first; waves skip key tiles that lie wholly
//    above their queries' diagonal.
//  * Key pieces (the _ws entry points): a causal chunk's query tiles carry
//    unequal work (tile t attends about p0 + 128(t+1) keys), and a short prompt
//    has too few workgroups to keep the device busy while its heaviest tiles
//    finish. Tiles with more key tiles than their share of the device's
//    workgroup slots are cut into up to four key ranges, one workgroup each;
//    every piece publishes its unnormalised (o, m, l), and the last piece of the
//    (tile, Q head) to arrive merges them in piece order.
#include <algorithm>
#include <cmath>
#include <type_traits>
#include <vector>

#include "af_common.h"
#include "af_device.h"

namespace af {
namespace {

constexpr int kPfHd = 128;
constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfKeys = 64;                      // keys per LDS tile
constexpr int kTileBytes = kPfKeys * kPfHd * 2;  // one K or V tile: 64 rows of 256 B
constexpr float kPfSumLimit = 256.0f;  // per-lane tile row sum that forces a rescale
constexpr float kPfEmptyMax = -1e30f;
constexpr int kPfQueries = 32 * kPfWaves;  // queries per workgroup (query tile)
constexpr int kPfMaxPieces = 4;            // key pieces per query tile
constexpr int kPfMinPieceTiles = 12;       // 64-key tiles per piece, at least

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

struct PrefillArgs {
    const uint16_t* q;   // query row i at q + i*q_stride, head h at +h*head_dim
    int64_t q_stride;
    const uint16_t* k;   // cache row t at k + t*kv_stride
    const uint16_t* v;
    int64_t kv_stride;
    uint32_t kv_row_bytes;  // kv_stride * 2; the cache spans less than 4 GiB
    uint16_t* out;       // output row i at out + i*out_stride
    int64_t out_stride;
    int32_t p0;
    int32_t n;
    int32_t kv_len;
    int32_t n_q_heads;
    int32_t n_kv_heads;
    int32_t n_tiles;     // ceil(n / queries per workgroup)
    float scale_log2;    // log2(e) / sqrt(head_dim)
    // Paged pool: k / v are the layer's K / V slabs (rows of kv_stride elements),
    // logical row t lives in slot table[t >> bs_log2] * block_size + t % block_size.
    const int32_t* table;
    int32_t bs_log2;
    int32_t max_block;  // table entries are clamped to [0, max_block] (the pool's last block)
    // FP8 pools: this layer's fp32 scales [2][n_kv_heads] (K, V); the slabs hold
    // E4M3 codes (one byte per element).
    const float* scales;
    // Batched chunks: workgroup tile tt handles query tile tile_map[2tt+1] of chunk
    // c = tile_map[2tt], chunks[4c..4c+3] = (p0, n, kv_len, first row in q / out),
    // block table at table + c * max_blocks. NULL: one chunk described above.
    const int32_t* tile_map;
    const int32_t* chunks;
    int32_t max_blocks;
    // Shared-prefix partials (part_o != NULL): the queries are the decode
    // tokens of many sequences, packed per KV head — query row i is sequence
    // i / q_group, Q head kv_head * q_group + i % q_group (n_q_heads is set to
    // n_kv_heads) — and every query sees all kv_len keys (p0 = kv_len). The
    // key tiles are split key_splits ways (workgroup id / (n_tiles * n_kv_heads)
    // is the split), and each (query, split) leaves an unnormalised partial in
    // the decode kernel's split-K record layout instead of an output row:
    //   part_o [seq][kv_head][rec_stride][q_group * 128] = o * v_scale
    //   part_ml[seq][kv_head][rec_stride][2 * q_group]   = (m, l), m in log2 units
    // at record index = split.
    int32_t q_group;
    int32_t key_splits;
    int32_t rec_stride;
    float* part_o;
    float* part_ml;
    // Partials with RoPE (cos_t != NULL): query rows hold pre-RoPE values and
    // sequence s is rotated at positions[s] (clamped into [0, max_pos)).
    const float* cos_t;
    const float* sin_t;
    const int32_t* positions;
    int32_t max_pos;
    // Key pieces (n_pieces > 1; single chunk, no tile map, no partials): query
    // tile t's key tiles are cut into min(n_pieces, ceil(tiles / piece_units))
    // balanced ranges, workgroup id / (n_kv_heads * group) % n_pieces being the
    // piece. A piece leaves its unnormalised output in
    //   rec_o [tile][q head][piece][128 x 128] (in the lanes' register order)
    //   rec_ml[tile][q head][piece][2][128 queries] = (m, l), m in log2 units
    // and takes counters[tile * n_q_heads + q head]; the last arrival merges the
    // pieces into the output and re-zeroes the counter.
    int32_t n_pieces;
    int32_t piece_units;
    // Batched chunks with key pieces: tile_map entries are 4 ints, (chunk, tile,
    // piece | pieces << 8, record group g); the pieces' records and counter
    // are those of tile index g (as tile above), n_pieces the most pieces.
    int32_t piece_map;
    float* rec_o;
    float* rec_ml;
    uint32_t* counters;
};

// Byte offset of 16-byte chunk `chunk` (0..15) of row `row` in a K tile.
__device__ __forceinline__ uint32_t k_off(int row, int chunk) {
    return uint32_t(row) * 256u + 16u * uint32_t(chunk ^ (row & 15));
}
// Same in a V tile.
__device__ __forceinline__ uint32_t v_off(int row, int chunk) {
    return uint32_t(row) * 256u + 16u * uint32_t(chunk ^ (4 * (row & 3)));
}

__device__ __forceinline__ uint4 ld16(const uint16_t* p) {
    return *reinterpret_cast<const uint4*>(p);
}

// Loads one 64-key K or V tile straight into LDS (global_load_lds_dwordx4: lane
// l of a wave writes the 16 bytes at LDS base + 16*l). Wave w fills rows
// 16w .. 16w+15, four rows per instruction; the lane at physical chunk p of row r
// fetches logical chunk p ^ swz(r), which realises the swizzled layout. Rows past
// kv_len load row kv_len-1: finite data whose scores are masked. base: the
// head's first element in cache row (slot) 0, as bytes. Contiguous caches use
// 32-bit row offsets (scalar base + vector offset); paged pools map the row
// through blk[i], the physical block of the lane's row in instruction i.
template <bool IS_K, bool PAGED>
__device__ __forceinline__ void dma_tile(const char* base, uint32_t row_bytes, int key0,
                                         int kv_len, int wave, int lane, char* lds_tile,
                                         const int (&blk)[4], int bs_log2) {
    const int pr = lane >> 4, pc = lane & 15;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 16 * wave + 4 * i + pr;  // tile row
        const int chunk = IS_K ? (pc ^ (r & 15)) : (pc ^ (4 * (r & 3)));
        const int key = min(key0 + r, kv_len - 1);
        const char* src;
        if constexpr (PAGED) {
            const int64_t slot = (int64_t(blk[i]) << bs_log2) | (key & ((1 << bs_log2) - 1));
            src = base + slot * row_bytes + 16 * chunk;
        } else {
            src = base + (__umul24(uint32_t(key), row_bytes) + 16u * chunk);
        }
        __builtin_amdgcn_global_load_lds(
            src, (__attribute__((address_space(3))) void*)(lds_tile + (16 * wave + 4 * i) * 256),
            16, 0, 0);
    }
}

// Physical blocks of the rows this lane fetches for tile `kt` (paged pools).
__device__ __forceinline__ void tile_blocks(const int32_t* table, int bs_log2, int max_block, int kt,
                                            int kv_len, int wave, int lane, int (&blk)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int key = min(kt * kPfKeys + 16 * wave + 4 * i + (lane >> 4), kv_len - 1);
        blk[i] = min(max(table[key >> bs_log2], 0), max_block);  // never address outside the pool
    }
}

// Physical block of logical row `key` (paged pools), clamped to the pool.
__device__ __forceinline__ int table_block(const PrefillArgs& a, int key) {
    return min(max(a.table[key >> a.bs_log2], 0), a.max_block);
}

// FP8 pools: tile rows go through registers, 32 codes of K and of V per thread
// (row tid/4, elements 32*(tid%4) ..), converted to fp16 exactly (E4M3 -> fp16,
// unit scale) after the current tile's matrix work and stored in the same
// swizzled layout as the DMA path. The K/V scales are applied to the scores and
// the output instead.
struct Fp8Tile {
    uint4 k0, k1, v0, v1;
};

template <bool PAGED>
__device__ __forceinline__ void fp8_load(const char* kb, const char* vb, uint32_t row_bytes,
                                         int key0, int kv_len, int tid, int blk, int bs_log2,
                                         Fp8Tile& t) {
    const int key = min(key0 + (tid >> 2), kv_len - 1);
    const int64_t slot =
        PAGED ? ((int64_t(blk) << bs_log2) | (key & ((1 << bs_log2) - 1))) : int64_t(key);
    const size_t off = size_t(slot) * row_bytes + 32 * (tid & 3);
    t.k0 = *reinterpret_cast<const uint4*>(kb + off);
    t.k1 = *reinterpret_cast<const uint4*>(kb + off + 16);
    t.v0 = *reinterpret_cast<const uint4*>(vb + off);
    t.v1 = *reinterpret_cast<const uint4*>(vb + off + 16);
}

// Eight E4M3 codes (two words) -> eight fp16 values.
__device__ __forceinline__ uint4 e4m3x8_to_f16(uint32_t w0, uint32_t w1) {
    uint4 r;
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(w0), 1.0f, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(w0), 1.0f, true));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(w1), 1.0f, false));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(w1), 1.0f, true));
    return r;
}

__device__ __forceinline__ void fp8_store(char* ks, char* vs, int tid, const Fp8Tile& t) {
    const int row = tid >> 2, q = tid & 3;
    // chunk 4q + c holds elements 32q + 8c .. +7
    *reinterpret_cast<uint4*>(ks + k_off(row, 4 * q + 0)) = e4m3x8_to_f16(t.k0.x, t.k0.y);
    *reinterpret_cast<uint4*>(ks + k_off(row, 4 * q + 1)) = e4m3x8_to_f16(t.k0.z, t.k0.w);
    *reinterpret_cast<uint4*>(ks + k_off(row, 4 * q + 2)) = e4m3x8_to_f16(t.k1.x, t.k1.y);
    *reinterpret_cast<uint4*>(ks + k_off(row, 4 * q + 3)) = e4m3x8_to_f16(t.k1.z, t.k1.w);
    // V's swizzle permutes whole 64-B chunk groups by row % 4, so the same store
    // of rows r and r + 1 would meet in the same banks (counters: 0.67 conflicts
    // per LDS access). Each lane stores its four chunks rotated by row % 4, so
    // one instruction's rows land in different 16-B bank groups.
    const uint4 c0 = e4m3x8_to_f16(t.v0.x, t.v0.y), c1 = e4m3x8_to_f16(t.v0.z, t.v0.w);
    const uint4 c2 = e4m3x8_to_f16(t.v1.x, t.v1.y), c3 = e4m3x8_to_f16(t.v1.z, t.v1.w);
    const int rot = row & 3;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int cc = (c + rot) & 3;
        const uint4 val = cc == 0 ? c0 : cc == 1 ? c1 : cc == 2 ? c2 : c3;
        *reinterpret_cast<uint4*>(vs + v_off(row, 4 * q + cc)) = val;
    }
}

__device__ __forceinline__ half8 lds_half8(const char* p) {
    return __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(p));
}

// V^T operand of one (16-key step, 32-d block): two transposing reads of 4 keys.
__device__ __forceinline__ half8 lds_vt(const char* p0, const char* p1) {
    typedef short4_t __attribute__((address_space(3)))* lds_s4;
    const short4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(p0));
    const short4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(p1));
    typedef short short8_t __attribute__((ext_vector_type(8)));
    const short8_t r = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(half8, r);
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

__device__ __forceinline__ float dot2_sum(const half8& h, float acc) {
    typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
    const half2_t one = {f16(1.0f), f16(1.0f)};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const half2_t p = {h[2 * t], h[2 * t + 1]};
        acc = __builtin_amdgcn_fdot2(p, one, acc, false);
    }
    return acc;
}

// LDS: K tiles at [0, 2*kTileBytes), V tiles after them.
constexpr int kVBase = 2 * kTileBytes;

__device__ __forceinline__ void store_agent2(uint64_t* p, float x, float y) {
    const auto u = [](float f) { return uint64_t(__builtin_bit_cast(uint32_t, f)); };
    __hip_atomic_store(p, u(x) | (u(y) << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float2 load_agent2(const uint64_t* p) {
    const uint64_t a = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__builtin_bit_cast(float, uint32_t(a)), __builtin_bit_cast(float, uint32_t(a >> 32)));
}

// End of a key piece: publish (o, m, l) of this workgroup's queries, arrive at
// the (tile, Q head) counter, and, in the last piece to arrive, merge every
// piece in piece order (own piece from registers: the bits it stored) and write
// the output. Publication relies on gfx950 rules, not on the language's
// relaxed atomics: agent-scope stores (sc1) write through to where every XCD
// reads; s_waitcnt vmcnt(0) covers stores on gfx9, so each wave's records are
// acknowledged before the barrier; the barrier orders them before the one
// returning agent-scope atomic; the merging workgroup's agent-scope loads are
// issued after the barrier that publishes that atomic's result. Lane (col, hi)
// holds query t0 + 32 wave + col at dims 32 db + 8 (r / 4) + 4 hi + r % 4 of
// o[db][r], and m / l of its query (the same in lanes col and col + 32). A
// piece's o record is kept in that register order, o[db][2i .. 2i+1] of lane l
// of wave w at 64-bit word (w * 32 + db * 8 + i) * 64 + l, so each store and
// load instruction covers 512 contiguous bytes; the merging workgroup's lanes
// hold the same queries and dims.
__device__ __forceinline__ void merge_pieces(const PrefillArgs& a, float16v (&o)[4], float m_run,
                                          float l_run, int tile, int head, int piece, int pieces,
                                          int t0, int wq0, bool wave_live, float v_scale) {
    __shared__ uint32_t s_arrived;
    const int tid = threadIdx.x, lane = tid & 63;
    const int col = lane & 31, hi = lane >> 5;
    const int qi = wq0 + col;
    const bool valid = wave_live && qi < a.n;
    const float l_sum = halves_sum(l_run);
    const int qrow = qi - t0;  // 0 .. 127
    const size_t grp = size_t(tile) * a.n_q_heads + head;
    const size_t rec0 = grp * a.n_pieces;
    constexpr size_t kRecO = size_t(kPfQueries) * kPfHd, kRecMl = 2 * kPfQueries;
    // this lane's first 64-bit word in a piece's o record
    const size_t lane_word = size_t(tid >> 6) * 32 * 64 + lane;
    if (valid) {
        uint64_t* ro = reinterpret_cast<uint64_t*>(a.rec_o + (rec0 + piece) * kRecO) + lane_word;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                store_agent2(ro + (db * 8 + i) * 64, o[db][2 * i], o[db][2 * i + 1]);
        if (hi == 0) {
            float* ml = a.rec_ml + (rec0 + piece) * kRecMl;
            __hip_atomic_store(ml + qrow, m_run, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ml + kPfQueries + qrow, l_sum, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
        s_arrived = __hip_atomic_fetch_add(a.counters + grp, 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_arrived != uint32_t(pieces - 1)) return;
    if (tid == 0) __hip_atomic_store(a.counters + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!valid) return;
    float mp[kPfMaxPieces], lp[kPfMaxPieces];
#pragma unroll
    for (int p = 0; p < kPfMaxPieces; ++p) {
        mp[p] = kPfEmptyMax;
        lp[p] = 0.0f;
        if (p < pieces) {
            if (p == piece) {
                mp[p] = m_run;
                lp[p] = l_sum;
            } else {
                const float* ml = a.rec_ml + (rec0 + p) * kRecMl;
                mp[p] = __hip_atomic_load(ml + qrow, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                lp[p] = __hip_atomic_load(ml + kPfQueries + qrow, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    float mx = mp[0];
#pragma unroll
    for (int p = 1; p < kPfMaxPieces; ++p) mx = fmaxf(mx, mp[p]);
    float wp[kPfMaxPieces], lt = 0.0f;
#pragma unroll
    for (int p = 0; p < kPfMaxPieces; ++p) {
        wp[p] = p < pieces ? fast_exp2(mp[p] - mx) : 0.0f;  // 0 for a piece without keys
        lt = fmaf(wp[p], lp[p], lt);
    }
    const float inv = v_scale / lt;
    uint16_t* orow = a.out + size_t(qi) * a.out_stride + size_t(head) * kPfHd + 4 * hi;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        float16v acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int p = 0; p < kPfMaxPieces; ++p) {
            if (p >= pieces) continue;
            if (p == piece) {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] = fmaf(wp[p], o[db][r], acc[r]);
            } else {
                const uint64_t* src = reinterpret_cast<const uint64_t*>(a.rec_o + (rec0 + p) * kRecO) +
                                      lane_word + db * 8 * 64;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float2 x = load_agent2(src + i * 64);
                    acc[2 * i] = fmaf(wp[p], x.x, acc[2 * i]);
                    acc[2 * i + 1] = fmaf(wp[p], x.y, acc[2 * i + 1]);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint2 w;
            w.x = uint32_t(f2h(acc[4 * g] * inv)) | (uint32_t(f2h(acc[4 * g + 1] * inv)) << 16);
            w.y = uint32_t(f2h(acc[4 * g + 2] * inv)) | (uint32_t(f2h(acc[4 * g + 3] * inv)) << 16);
            *reinterpret_cast<uint2*>(orow + 32 * db + 8 * g) = w;
        }
    }
}

template <bool PAGED, bool FP8>
__global__ __launch_bounds__(kPfThreads, 2) void prefill_attention_kernel(const PrefillArgs args) {
    PrefillArgs a = args;
    constexpr int kQueries = 32 * kPfWaves;  // per workgroup
    __shared__ __align__(16) char s_lds[4 * kTileBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform branches below
    const int col = lane & 31, hi = lane >> 5;
    // Block order: KV head fastest, then Q head of the group, then query tile
    // heaviest first.
    const int group = a.n_q_heads / a.n_kv_heads;
    int bid = int(blockIdx.x);
    int ks = 0;     // key split (shared-prefix partials)
    int piece = 0;  // key piece
    if (a.part_o) {
        const int per = a.n_tiles * a.n_q_heads;
        ks = bid / per;
        bid -= ks * per;
    }
    const int kvh = bid % a.n_kv_heads;
    const int rest = bid / a.n_kv_heads;
    const int head = kvh * group + rest % group;
    int tile;
    int map_pieces = 0, rec_tile = 0;  // batched key pieces: from the map
    if (a.tile_map) {  // batched chunks: the host orders the tiles heaviest first
        const int tt = rest / group;
        const int es = a.piece_map ? 4 : 2;
        const int c = __builtin_amdgcn_readfirstlane(a.tile_map[es * tt]);
        tile = __builtin_amdgcn_readfirstlane(a.tile_map[es * tt + 1]);
        if (a.piece_map) {
            const int pp = __builtin_amdgcn_readfirstlane(a.tile_map[4 * tt + 2]);
            piece = pp & 0xff;
            map_pieces = pp >> 8;
            rec_tile = __builtin_amdgcn_readfirstlane(a.tile_map[4 * tt + 3]);
        }
        const int32_t* ci = a.chunks + 4 * c;
        a.p0 = __builtin_amdgcn_readfirstlane(ci[0]);
        a.n = __builtin_amdgcn_readfirstlane(ci[1]);
        a.kv_len = __builtin_amdgcn_readfirstlane(ci[2]);
        const int row0 = __builtin_amdgcn_readfirstlane(ci[3]);
        a.q += size_t(row0) * a.q_stride;
        a.out += size_t(row0) * a.out_stride;
        a.table += size_t(c) * a.max_blocks;
    } else if (a.n_pieces > 1) {  // key pieces: the pieces of a tile are adjacent
        const int r2 = rest / group;
        piece = r2 % a.n_pieces;
        tile = a.n_tiles - 1 - r2 / a.n_pieces;
    } else {
        tile = a.n_tiles - 1 - rest / group;
    }
    const int t0 = tile * kQueries;
    const int wq0 = t0 + 32 * wave;  // the wave's first query
    const bool wave_live = wq0 < a.n;

    const int wg_keys = min(a.p0 + min(t0 + kQueries, a.n), a.kv_len);
    // Key tiles [kt_lo, n_kt) of this workgroup: all of them, or one key split's.
    int kt_lo = 0, n_kt = (wg_keys + kPfKeys - 1) / kPfKeys;
    if (a.part_o) {
        const int all = n_kt;
        kt_lo = ks * all / a.key_splits;
        n_kt = (ks + 1) * all / a.key_splits;
    }
    int pieces = 1;  // workgroup-uniform
    if (a.n_pieces > 1) {
        const int all = n_kt;
        if (a.piece_map) {  // the host planned this tile's pieces (at most its key tiles)
            pieces = min(map_pieces, all);
        } else {
            pieces = min(a.n_pieces, (all + a.piece_units - 1) / a.piece_units);
            rec_tile = tile;
        }
        if (piece >= pieces) return;  // a lighter tile needs fewer pieces
        kt_lo = piece * all / pieces;
        n_kt = (piece + 1) * all / pieces;
    }
    // Keys the wave needs.
    const int w_keys = wave_live ? min(a.p0 + min(wq0 + 32, a.n), a.kv_len) : 0;

    // Query operands first: the loop's first waits then cover them.
    half8 qf[8];
    const int qi_lane = min(wq0 + col, a.n - 1);  // clamped
    const int lim = min(a.p0 + qi_lane + 1, a.kv_len);     // this lane's query attends [0, lim)
    const int mask_from = min(a.p0 + wq0 + 1, a.kv_len);  // first key hidden from some query
    // Packed partials with RoPE: this lane's (dim, dim + 64) pairs are qf[s][t],
    // qf[s + 4][t] at dim 16s + 8hi + t (s < 4); their cos / sin go in flight here.
    float4 rope_c[8], rope_s[8];
    {
        const uint16_t* qrow;
        if (a.q_group) {
            const int sq = qi_lane / a.q_group;
            qrow = a.q + size_t(sq) * a.q_stride +
                   size_t(head * a.q_group + qi_lane - sq * a.q_group) * kPfHd + 8 * hi;
            if (a.cos_t) {
                const int pos = min(max(a.positions[sq], 0), a.max_pos - 1);
                const float* cr = a.cos_t + size_t(pos) * (kPfHd / 2) + 8 * hi;
                const float* sr = a.sin_t + size_t(pos) * (kPfHd / 2) + 8 * hi;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    rope_c[2 * s] = *reinterpret_cast<const float4*>(cr + 16 * s);
                    rope_c[2 * s + 1] = *reinterpret_cast<const float4*>(cr + 16 * s + 4);
                    rope_s[2 * s] = *reinterpret_cast<const float4*>(sr + 16 * s);
                    rope_s[2 * s + 1] = *reinterpret_cast<const float4*>(sr + 16 * s + 4);
                }
            }
        } else {
            qrow = a.q + size_t(qi_lane) * a.q_stride + size_t(head) * kPfHd + 8 * hi;
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) qf[s] = __builtin_bit_cast(half8, ld16(qrow + 16 * s));
    }
    // Keep the query loads ahead of the tile loads: the prologue's wait for the
    // tile then covers them, and the loop never waits on a query register.
    asm volatile("" ::: "memory");
    constexpr int kElem = FP8 ? 1 : 2;
    const char* kb = reinterpret_cast<const char*>(a.k) + size_t(kvh) * kPfHd * kElem;
    const char* vb = reinterpret_cast<const char*>(a.v) + size_t(kvh) * kPfHd * kElem;
    // Paged: the block-table entries of tile kt+1 are loaded one step ahead, so
    // the wait for tile kt's data also covers them.
    int blk[4] = {0, 0, 0, 0};
    int blk8 = 0;  // FP8: this thread's row's block for the next tile
    Fp8Tile f8;
    const int key_lo = kt_lo * kPfKeys;
    if constexpr (FP8) {
        if constexpr (PAGED) blk8 = table_block(a, min(key_lo + (tid >> 2), a.kv_len - 1));
        fp8_load<PAGED>(kb, vb, a.kv_row_bytes, key_lo, a.kv_len, tid, blk8, a.bs_log2, f8);
        fp8_store(s_lds, s_lds + kVBase, tid, f8);
        if constexpr (PAGED)
            if (kt_lo + 1 < n_kt)
                blk8 = table_block(a, min(key_lo + kPfKeys + (tid >> 2), a.kv_len - 1));
    } else {
        if constexpr (PAGED)
            tile_blocks(a.table, a.bs_log2, a.max_block, kt_lo, a.kv_len, wave, lane, blk);
        dma_tile<true, PAGED>(kb, a.kv_row_bytes, key_lo, a.kv_len, wave, lane, s_lds, blk,
                              a.bs_log2);
        dma_tile<false, PAGED>(vb, a.kv_row_bytes, key_lo, a.kv_len, wave, lane, s_lds + kVBase,
                               blk, a.bs_log2);
        if constexpr (PAGED)
            if (kt_lo + 1 < n_kt)
                tile_blocks(a.table, a.bs_log2, a.max_block, kt_lo + 1, a.kv_len, wave, lane, blk);
    }
    if (a.cos_t) {  // packed partials with RoPE (wave-uniform)
        // Whole 32-bit words in and out: two fp16 elements per word, low half
        // first. (Element-wise read-modify-write of the half8 vectors compiled
        // to code that fed each rotated element into the next pair.)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint4 xw = __builtin_bit_cast(uint4, qf[s]);
            const uint4 yw = __builtin_bit_cast(uint4, qf[s + 4]);
            const uint32_t xs[4] = {xw.x, xw.y, xw.z, xw.w};
            const uint32_t ys[4] = {yw.x, yw.y, yw.z, yw.w};
            const float cs[8] = {rope_c[2 * s].x, rope_c[2 * s].y, rope_c[2 * s].z,
                                 rope_c[2 * s].w, rope_c[2 * s + 1].x, rope_c[2 * s + 1].y,
                                 rope_c[2 * s + 1].z, rope_c[2 * s + 1].w};
            const float sn[8] = {rope_s[2 * s].x, rope_s[2 * s].y, rope_s[2 * s].z,
                                 rope_s[2 * s].w, rope_s[2 * s + 1].x, rope_s[2 * s + 1].y,
                                 rope_s[2 * s + 1].z, rope_s[2 * s + 1].w};
            uint32_t xo[4], yo[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint16_t x0, y0, x1, y1;
                rope_rotate(uint16_t(xs[w] & 0xffffu), uint16_t(ys[w] & 0xffffu), cs[2 * w],
                            sn[2 * w], x0, y0);
                rope_rotate(uint16_t(xs[w] >> 16), uint16_t(ys[w] >> 16), cs[2 * w + 1],
                            sn[2 * w + 1], x1, y1);
                xo[w] = uint32_t(x0) | (uint32_t(x1) << 16);
                yo[w] = uint32_t(y0) | (uint32_t(y1) << 16);
            }
            qf[s] = __builtin_bit_cast(half8, make_uint4(xo[0], xo[1], xo[2], xo[3]));
            qf[s + 4] = __builtin_bit_cast(half8, make_uint4(yo[0], yo[1], yo[2], yo[3]));
        }
    }

    // Per-lane LDS operand offsets; the buffer, the key block and the key step
    // are added as immediates.
    //  K: row col (+32 for keys 32..63), chunk 2s+hi.
    //  V^T: lane l of 16-lane group G reads row K0 + (l%16)/4 at d = 32db +
    //  16(G%2) + 4(l%4), K0 = 16j + 8u + 4hi (u: first / second four slots).
    uint32_t ka[8], va[4];
#pragma unroll
    for (int s = 0; s < 8; ++s) ka[s] = k_off(col, 2 * s + hi);
    {
        const int jl = lane & 15, g1 = (lane >> 4) & 1;
        const int rl = jl >> 2;  // row within the 4-key group (= row % 4)
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int d = 32 * db + 16 * g1 + 4 * (jl & 3);
            va[db] = kVBase + v_off(4 * hi + rl, d >> 3) + 2 * (d & 7);
        }
    }

    float16v o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    float m_run = kPfEmptyMax, l_run = 0.0f;
    // FP8: scores carry the K scale, the output the V scale.
    const float sc = FP8 ? a.scale_log2 * a.scales[kvh] : a.scale_log2;
    const float v_scale = FP8 ? a.scales[a.n_kv_heads + kvh] : 1.0f;

    auto step = [&](int kt, auto buf_c) {
        constexpr int BUF = decltype(buf_c)::value;
        // This wave's tile loads have landed in LDS; the barrier covers the others'
        // and frees the other buffer (read in the previous step) for the next tile.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (kt + 1 < n_kt) {
            if constexpr (FP8) {
                fp8_load<PAGED>(kb, vb, a.kv_row_bytes, (kt + 1) * kPfKeys, a.kv_len, tid, blk8,
                                a.bs_log2, f8);
                if constexpr (PAGED)
                    if (kt + 2 < n_kt)
                        blk8 = table_block(a, min((kt + 2) * kPfKeys + (tid >> 2), a.kv_len - 1));
            } else {
                dma_tile<true, PAGED>(kb, a.kv_row_bytes, (kt + 1) * kPfKeys, a.kv_len, wave, lane,
                                      s_lds + (BUF ^ 1) * kTileBytes, blk, a.bs_log2);
                dma_tile<false, PAGED>(vb, a.kv_row_bytes, (kt + 1) * kPfKeys, a.kv_len, wave,
                                       lane, s_lds + kVBase + (BUF ^ 1) * kTileBytes, blk,
                                       a.bs_log2);
                if constexpr (PAGED)
                    if (kt + 2 < n_kt)
                        tile_blocks(a.table, a.bs_log2, a.max_block, kt + 2, a.kv_len, wave, lane,
                                    blk);
            }
        }
        const int key0 = kt * kPfKeys;
        const char* ks = s_lds + BUF * kTileBytes;
        const char* vs = s_lds + BUF * kTileBytes;  // va[] carries the V region's base
        // Two halves of 32 keys: QK^T, softmax, then P.V for each.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int keyh = key0 + 32 * kb;
            if (keyh >= w_keys) break;  // wave-uniform
            float16v sacc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const half8 kf = lds_half8(ks + ka[s] + kb * 32 * 256);
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], sacc, 0, 0, 0);
            }
            // Register r holds key keyh + 8(r/4) + 4hi + r%4.
            if (keyh + 32 > mask_from) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = keyh + 8 * (r >> 2) + 4 * hi + (r & 3);
                    sacc[r] = key < lim ? sacc[r] : -INFINITY;
                }
            }
            // Probabilities against the running max m_run, rounded to fp16, and
            // their row sum. While each lane's sum stays <= 2^8, every p is <= 2^8
            // and m_run is kept (it may trail the true max by up to 8 in log2
            // units; fp16 holds p to 2^15). Otherwise (the first keys, or scores
            // that grew) the exact running max is taken and O^T, l rescaled: the
            // max is computed only on this path.
            half8 pj[2];
            float ls;
            auto probs = [&]() {
                float16v pv;
#pragma unroll
                for (int r = 0; r < 16; ++r) pv[r] = fast_exp2(fmaf(sacc[r], sc, -m_run));
                pj[0] = to_half8(pv, 0);
                pj[1] = to_half8(pv, 8);
                ls = dot2_sum(pj[1], dot2_sum(pj[0], 0.0f));
            };
            probs();
            if (__builtin_amdgcn_ballot_w64(!(ls <= kPfSumLimit))) {
                float mx = sacc[0];
#pragma unroll
                for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sacc[r]);
                const float m_new = fmaxf(m_run, halves_max(mx) * sc);
                const float alpha = fast_exp2(m_run - m_new);
                m_run = m_new;
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
                probs();
            }
            l_run += ls;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const char* p = vs + va[db] + 16 * (2 * kb + jj) * 256;
                    const half8 vt = lds_vt(p, p + 8 * 256);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vt, pj[jj], o[db], 0, 0, 0);
                }
        }
        if constexpr (FP8)
            if (kt + 1 < n_kt)
                fp8_store(s_lds + (BUF ^ 1) * kTileBytes, s_lds + kVBase + (BUF ^ 1) * kTileBytes,
                          tid, f8);
    };
    int kt = kt_lo;
    for (; kt + 2 <= n_kt; kt += 2) {
        step(kt, std::integral_constant<int, 0>{});
        step(kt + 1, std::integral_constant<int, 1>{});
    }
    if (kt < n_kt) step(kt, std::integral_constant<int, 0>{});

    if (pieces > 1) {
        merge_pieces(a, o, m_run, l_run, rec_tile, head, piece, pieces, t0, wq0, wave_live, v_scale);
        return;
    }
    if (!wave_live) return;
    const int qi = wq0 + col;
    const float l_sum = halves_sum(l_run);
    if (qi >= a.n) return;
    if (a.part_o) {  // shared-prefix partial: (o * v_scale, m, l) of split ks
        const int sq = qi / a.q_group, gh = qi - sq * a.q_group;
        const size_t rec = (size_t(sq) * a.n_kv_heads + kvh) * a.rec_stride + ks;
        float* po = a.part_o + rec * (size_t(a.q_group) * kPfHd) + gh * kPfHd + 4 * hi;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<float4*>(po + 32 * db + 8 * g) =
                    make_float4(o[db][4 * g] * v_scale, o[db][4 * g + 1] * v_scale,
                                o[db][4 * g + 2] * v_scale, o[db][4 * g + 3] * v_scale);
        if (hi == 0) {
            float* ml = a.part_ml + rec * 2 * a.q_group;
            ml[gh] = m_run;
            ml[a.q_group + gh] = l_sum;
        }
        return;
    }
    const float inv = v_scale / l_sum;
    uint16_t* orow = a.out + size_t(qi) * a.out_stride + size_t(head) * kPfHd + 4 * hi;
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

int launch_prefill(PrefillArgs a, hipStream_t stream) {
    a.n_tiles = ceil_div(a.n, 32 * kPfWaves);
    const dim3 grid(a.n_tiles * a.n_q_heads * std::max(a.n_pieces, 1)), block(kPfThreads);
    if (a.scales)
        hipLaunchKernelGGL((prefill_attention_kernel<true, true>), grid, block, 0, stream, a);
    else if (a.table)
        hipLaunchKernelGGL((prefill_attention_kernel<true, false>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((prefill_attention_kernel<false, false>), grid, block, 0, stream, a);
    AF_TRY_LAUNCH();
    return AF_OK;
}

}  // namespace

int prefix_partial_tiles(int batch, int group, int n_kv_heads) {
    return ceil_div(batch * group, 32 * kPfWaves) * n_kv_heads;
}

int launch_prefix_partials(const PrefixPartialArgs& p, hipStream_t stream) {
    PrefillArgs a{};
    a.q = p.q;
    a.q_stride = p.q_stride;
    a.k = reinterpret_cast<const uint16_t*>(p.k);
    a.v = reinterpret_cast<const uint16_t*>(p.v);
    a.kv_stride = int64_t(p.n_kv_heads) * kPfHd;
    a.kv_row_bytes = uint32_t(p.row_bytes);
    a.n = p.batch * p.group;  // packed: one query per (sequence, Q head of the group)
    a.p0 = p.prefix_len;      // every query follows the whole prefix
    a.kv_len = p.prefix_len;
    a.n_q_heads = p.n_kv_heads;
    a.n_kv_heads = p.n_kv_heads;
    a.n_tiles = ceil_div(a.n, 32 * kPfWaves);
    a.scale_log2 = float(1.4426950408889634 / std::sqrt(double(kPfHd)));
    a.table = p.table;
    a.bs_log2 = p.bs_log2;
    a.max_block = int32_t(std::min<int64_t>(p.total_blocks - 1, INT32_MAX));
    a.scales = p.scales;
    a.q_group = p.group;
    a.key_splits = p.key_splits;
    a.rec_stride = p.rec_stride;
    a.part_o = p.part_o;
    a.part_ml = p.part_ml;
    a.cos_t = p.cos_t;
    a.sin_t = p.sin_t;
    a.positions = p.positions;
    a.max_pos = p.max_pos;
    const dim3 grid(a.n_tiles * a.n_q_heads * p.key_splits), block(kPfThreads);
    if (p.scales)
        hipLaunchKernelGGL((prefill_attention_kernel<true, true>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((prefill_attention_kernel<true, false>), grid, block, 0, stream, a);
    AF_TRY_LAUNCH();
    return AF_OK;
}

// Key-tiles per piece for a launch whose query tiles need units[i] 64-key
// tiles each (times n_q_heads workgroups), or 0 for no cut. Only a grid with
// fewer workgroups than the device has slots (two per CU) is cut: a grid that
// fills the device is already balanced by its heaviest-first order, and cutting
// it only adds record traffic (MI355X: a 4096-token prompt 129 -> 143 us). A
// piece is about 1.6 slot shares of the launch's work (1.0 / 1.3 / 1.6 measured:
// a serving step's chunks 67 / 61 / 59 us, a 2048-token prompt 52 / 48 / 48 us),
// and at least kPfMinPieceTiles tiles (shorter pieces cost more in set-up and
// merge than they gain). Tile i then has min(cap, ceil(units[i] / per)) pieces.
// With `concurrent`, per also grows until every piece has a slot at once: the
// single-chunk grid orders pieces by tile, not by size, so a piece that waited
// for a slot could be a whole uncut tile queued behind smaller pieces.
int piece_tiles(const std::vector<int>& units, int n_q_heads, int cap, bool concurrent) {
    const int64_t slots = 2 * int64_t(device_compute_units());
    const int64_t tiles = int64_t(units.size());
    if (cap <= 1 || tiles == 0 || tiles * n_q_heads >= slots || tiles * n_q_heads > kMaxCounters)
        return 0;
    int64_t work = 0;
    int most = 0;
    for (int u : units) {
        work += u;
        most = std::max(most, u);
    }
    int per = int(std::max<int64_t>(kPfMinPieceTiles, (work * n_q_heads * 8 + 5 * slots - 1) /
                                                          (5 * slots)));
    auto wgs = [&](int pt) {
        int64_t w = 0;
        for (int u : units) w += std::min(cap, ceil_div(u, pt));
        return w * n_q_heads;
    };
    if (concurrent)
        while (per < most && wgs(per) > slots) ++per;
    return per < most ? per : 0;
}

// Key pieces of one chunk (piece_tiles over its query tiles). Returns the most
// pieces of any tile (1: no cut) and the tiles per piece in *units.
int plan_pieces(int p0, int n, int kv_len, int n_q_heads, int max_pieces, int* units) {
    *units = 0;
    const int nt = ceil_div(n, kPfQueries);
    if (n <= 0) return 1;
    std::vector<int> u(nt);
    int most = 0;
    for (int t = 0; t < nt; ++t) {
        const int keys = std::min(p0 + std::min((t + 1) * kPfQueries, n), kv_len);
        u[t] = ceil_div(std::max(keys, 1), kPfKeys);
        most = std::max(most, u[t]);
    }
    const int cap = std::min(max_pieces, kPfMaxPieces);
    const int per = piece_tiles(u, n_q_heads, cap, true);
    if (per == 0) return 1;
    const int pieces = std::min(cap, ceil_div(most, per));
    if (pieces <= 1) return 1;
    *units = per;
    return pieces;
}

// Workspace of a key-piece launch: the counter region of the attention
// workspaces (zero between launches), then rec_ml, then rec_o.
size_t record_workspace_bytes(int groups, int n_q_heads, int pieces) {
    if (pieces <= 1) return kCounterBytes;
    const size_t recs = size_t(groups) * n_q_heads * pieces;
    return kCounterBytes + align_up(recs * 2 * kPfQueries * sizeof(float), 256) +
           recs * kPfQueries * kPfHd * sizeof(float);
}

size_t piece_workspace_bytes(int n, int n_q_heads, int pieces) {
    return record_workspace_bytes(ceil_div(n, kPfQueries), n_q_heads, pieces);
}

void carve_records(PrefillArgs& a, void* workspace, int groups, int pieces) {
    char* w = static_cast<char*>(workspace);
    const size_t recs = size_t(groups) * a.n_q_heads * pieces;
    a.counters = reinterpret_cast<uint32_t*>(w);
    a.rec_ml = reinterpret_cast<float*>(w + kCounterBytes);
    a.rec_o = reinterpret_cast<float*>(w + kCounterBytes +
                                       align_up(recs * 2 * kPfQueries * sizeof(float), 256));
}

// Sets a's key pieces (key_pieces: 0 = plan_pieces' choice, 1 = none, else at
// most that many), checking the workspace.
int set_pieces(PrefillArgs& a, int key_pieces, void* workspace, size_t workspace_bytes) {
    if (key_pieces < 0 || key_pieces > kPfMaxPieces) return AF_ERR_INVALID_ARG;
    int units = 0;
    const int pieces = plan_pieces(a.p0, a.n, a.kv_len, a.n_q_heads,
                                   key_pieces == 0 ? kPfMaxPieces : key_pieces, &units);
    a.n_pieces = pieces;
    a.piece_units = units;
    if (pieces <= 1) return AF_OK;
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u) ||
        workspace_bytes < piece_workspace_bytes(a.n, a.n_q_heads, pieces))
        return AF_ERR_WORKSPACE;
    carve_records(a, workspace, ceil_div(a.n, kPfQueries), pieces);
    return AF_OK;
}

}  // namespace af

using namespace af;

// ---- b2 -----------------------------------------------------------------------
static int prefill_contig(const void* q, int q_stride, const void* k_cache, const void* v_cache,
                          void* out, int out_stride, int p0, int n, int kv_len, int max_seq,
                          int n_q_heads, int n_kv_heads, int head_dim, int key_pieces,
                          void* workspace, size_t workspace_bytes, af_stream_t stream) {
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
    // 32-bit row offsets in the kernel: the cache must span less than 4 GiB.
    if (int64_t(max_seq) * a.kv_stride * 2 >= (int64_t(1) << 32)) return AF_ERR_UNSUPPORTED;
    a.kv_row_bytes = uint32_t(a.kv_stride * 2);
    a.out = static_cast<uint16_t*>(out);
    a.out_stride = out_stride;
    a.p0 = p0;
    a.n = n;
    a.kv_len = kv_len;
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = n_kv_heads;
    a.scale_log2 = float(1.4426950408889634 / std::sqrt(double(head_dim)));
    if (int st = set_pieces(a, key_pieces, workspace, workspace_bytes)) return st;
    return launch_prefill(a, static_cast<hipStream_t>(stream));
}

extern "C" int af_prefill_attention(const void* q, int q_stride, const void* k_cache,
                                    const void* v_cache, void* out, int out_stride, int p0, int n,
                                    int kv_len, int max_seq, int n_q_heads, int n_kv_heads,
                                    int head_dim, af_stream_t stream) {
    return prefill_contig(q, q_stride, k_cache, v_cache, out, out_stride, p0, n, kv_len, max_seq,
                          n_q_heads, n_kv_heads, head_dim, 1, nullptr, 0, stream);
}

extern "C" int af_prefill_attention_ws(const void* q, int q_stride, const void* k_cache,
                                       const void* v_cache, void* out, int out_stride, int p0,
                                       int n, int kv_len, int max_seq, int n_q_heads,
                                       int n_kv_heads, int head_dim, int key_pieces,
                                       void* workspace, size_t workspace_bytes,
                                       af_stream_t stream) {
    return prefill_contig(q, q_stride, k_cache, v_cache, out, out_stride, p0, n, kv_len, max_seq,
                          n_q_heads, n_kv_heads, head_dim, key_pieces, workspace, workspace_bytes,
                          stream);
}

extern "C" size_t af_prefill_workspace_size(int p0, int n, int kv_len, int n_q_heads,
                                            int key_pieces) {
    if (p0 < 0 || n < 0 || n_q_heads <= 0 || key_pieces < 0 || key_pieces > kPfMaxPieces)
        return 0;
    int units = 0;
    const int pieces = plan_pieces(p0, n, kv_len, n_q_heads,
                                   key_pieces == 0 ? kPfMaxPieces : key_pieces, &units);
    return piece_workspace_bytes(n, n_q_heads, pieces);
}

static int prefill_paged(const void* q, int q_stride, const af_kv_pool* pool, int layer,
                         const int32_t* d_block_table, int max_blocks, int p0, int n, int kv_len,
                         void* out, int out_stride, int n_q_heads, int key_pieces, void* workspace,
                         size_t workspace_bytes, af_stream_t stream) {
    if (!q || !pool || !pool->base || !d_block_table || !out || n < 0 || p0 < 0 ||
        n_q_heads <= 0 || max_blocks <= 0)
        return AF_ERR_INVALID_ARG;
    if (layer < 0 || layer >= pool->n_layers || pool->n_kv_heads <= 0 ||
        n_q_heads % pool->n_kv_heads || pool->total_blocks <= 0 ||
        (pool->flags & ~AF_KV_POOL_SHARED_BLOCKS))
        return AF_ERR_INVALID_ARG;
    const bool fp8 = pool->dtype == AF_KV_FP8_E4M3;
    if ((!fp8 && pool->dtype != AF_KV_FP16) || pool->head_dim != kPfHd) return AF_ERR_UNSUPPORTED;
    if (fp8 && !pool->scales) return AF_ERR_INVALID_ARG;
    const int bs = pool->block_size;
    if (bs < 8 || (bs & (bs - 1))) return AF_ERR_INVALID_ARG;
    const int q_dim = n_q_heads * kPfHd;
    if (q_stride < q_dim || out_stride < q_dim || q_stride % 8 || out_stride % 8)
        return AF_ERR_INVALID_ARG;
    if (!aligned16(q) || !aligned16(out) || !aligned16(pool->base)) return AF_ERR_INVALID_ARG;
    if (n == 0) return AF_OK;
    if (kv_len <= 0 || int64_t(kv_len) > int64_t(max_blocks) * bs) return AF_ERR_OUT_OF_RANGE;
    const int64_t kv_stride = int64_t(pool->n_kv_heads) * kPfHd;
    const size_t esz = fp8 ? 1 : 2;
    const size_t slab = size_t(pool->total_blocks) * bs * kv_stride * esz;  // bytes
    const char* base = static_cast<const char*>(pool->base);
    PrefillArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.q_stride = q_stride;
    a.k = reinterpret_cast<const uint16_t*>(base + size_t(2 * layer) * slab);
    a.v = reinterpret_cast<const uint16_t*>(base + size_t(2 * layer + 1) * slab);
    a.kv_stride = kv_stride;
    a.kv_row_bytes = uint32_t(kv_stride * esz);
    a.scales = fp8 ? pool->scales + size_t(layer) * 2 * pool->n_kv_heads : nullptr;
    a.out = static_cast<uint16_t*>(out);
    a.out_stride = out_stride;
    a.p0 = p0;
    a.n = n;
    a.kv_len = kv_len;
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = pool->n_kv_heads;
    a.scale_log2 = float(1.4426950408889634 / std::sqrt(double(kPfHd)));
    a.table = d_block_table;
    a.bs_log2 = __builtin_ctz(unsigned(bs));
    a.max_block = int32_t(std::min<int64_t>(pool->total_blocks - 1, INT32_MAX));
    if (int st = set_pieces(a, key_pieces, workspace, workspace_bytes)) return st;
    return launch_prefill(a, static_cast<hipStream_t>(stream));
}

extern "C" int af_paged_prefill_attention(const void* q, int q_stride, const af_kv_pool* pool,
                                          int layer, const int32_t* d_block_table,
                                          int max_blocks, int p0, int n, int kv_len, void* out,
                                          int out_stride, int n_q_heads, af_stream_t stream) {
    return prefill_paged(q, q_stride, pool, layer, d_block_table, max_blocks, p0, n, kv_len, out,
                         out_stride, n_q_heads, 1, nullptr, 0, stream);
}

extern "C" int af_paged_prefill_attention_ws(const void* q, int q_stride, const af_kv_pool* pool,
                                             int layer, const int32_t* d_block_table,
                                             int max_blocks, int p0, int n, int kv_len, void* out,
                                             int out_stride, int n_q_heads, int key_pieces,
                                             void* workspace, size_t workspace_bytes,
                                             af_stream_t stream) {
    return prefill_paged(q, q_stride, pool, layer, d_block_table, max_blocks, p0, n, kv_len, out,
                         out_stride, n_q_heads, key_pieces, workspace, workspace_bytes, stream);
}

extern "C" int af_prefill_tile_map(const int32_t* h_chunks, int n_chunks, int32_t* h_tile_map,
                                   int max_tiles) {
    if (!h_chunks || !h_tile_map || n_chunks < 0 || max_tiles < 0) return AF_ERR_INVALID_ARG;
    struct T {
        int64_t work;
        int c, t;
    };
    std::vector<T> tiles;
    const int tq = 32 * kPfWaves;  // queries per tile of the launched kernel
    for (int c = 0; c < n_chunks; ++c) {
        const int p0 = h_chunks[4 * c], n = h_chunks[4 * c + 1], kv_len = h_chunks[4 * c + 2];
        if (p0 < 0 || n < 0 || h_chunks[4 * c + 3] < 0) return AF_ERR_INVALID_ARG;
        if (n > 0 && kv_len <= 0) return AF_ERR_OUT_OF_RANGE;
        for (int t = 0; t * tq < n; ++t) {
            const int64_t keys = std::min<int64_t>(int64_t(p0) + std::min((t + 1) * tq, n), kv_len);
            tiles.push_back({keys, c, t});
        }
    }
    if (int(tiles.size()) > max_tiles) return AF_ERR_WORKSPACE;
    std::stable_sort(tiles.begin(), tiles.end(), [](const T& x, const T& y) { return x.work > y.work; });
    for (size_t i = 0; i < tiles.size(); ++i) {
        h_tile_map[2 * i] = tiles[i].c;
        h_tile_map[2 * i + 1] = tiles[i].t;
    }
    return int(tiles.size());
}

extern "C" int af_prefill_piece_map(const int32_t* h_chunks, int n_chunks, int n_q_heads,
                                    int key_pieces, int32_t* h_map, int max_entries, int* n_groups,
                                    int* max_pieces, size_t* workspace_bytes) {
    if (!h_chunks || !h_map || !n_groups || !max_pieces || !workspace_bytes || n_chunks < 0 ||
        max_entries < 0 || n_q_heads <= 0 || key_pieces < 0 || key_pieces > kPfMaxPieces)
        return AF_ERR_INVALID_ARG;
    struct T {
        int units, c, t, g, pieces;
    };
    std::vector<T> tiles;
    for (int c = 0; c < n_chunks; ++c) {
        const int p0 = h_chunks[4 * c], n = h_chunks[4 * c + 1], kv_len = h_chunks[4 * c + 2];
        if (p0 < 0 || n < 0 || h_chunks[4 * c + 3] < 0) return AF_ERR_INVALID_ARG;
        if (n > 0 && kv_len <= 0) return AF_ERR_OUT_OF_RANGE;
        for (int t = 0; t * kPfQueries < n; ++t) {
            const int keys = std::min(p0 + std::min((t + 1) * kPfQueries, n), kv_len);
            const int u = ceil_div(std::max(keys, 1), kPfKeys);
            tiles.push_back({u, c, t, int(tiles.size()), 1});
        }
    }
    // piece_tiles over the launch's tiles; the map orders pieces by size, so
    // pieces may queue for slots.
    const int cap = key_pieces == 0 ? kPfMaxPieces : key_pieces;
    std::vector<int> units;
    for (const T& x : tiles) units.push_back(x.units);
    const int per = piece_tiles(units, n_q_heads, cap, false);
    int most = 1;
    if (per > 0)
        for (T& x : tiles) {
            x.pieces = std::min(cap, ceil_div(x.units, per));
            most = std::max(most, x.pieces);
        }
    // entries: every piece, heaviest piece first (a tile's pieces stay together)
    std::stable_sort(tiles.begin(), tiles.end(), [](const T& x, const T& y) {
        return int64_t(x.units) * y.pieces > int64_t(y.units) * x.pieces;
    });
    int n_entries = 0;
    for (const T& x : tiles) n_entries += x.pieces;
    if (n_entries > max_entries) return AF_ERR_WORKSPACE;
    int e = 0;
    for (const T& x : tiles)
        for (int p = 0; p < x.pieces; ++p, ++e) {
            h_map[4 * e] = x.c;
            h_map[4 * e + 1] = x.t;
            h_map[4 * e + 2] = p | (x.pieces << 8);
            h_map[4 * e + 3] = x.g;
        }
    *n_groups = int(tiles.size());
    *max_pieces = most;
    *workspace_bytes = record_workspace_bytes(int(tiles.size()), n_q_heads, most);
    return n_entries;
}

static int prefill_batched(const void* q, int q_stride, const af_kv_pool* pool, int layer,
                           const int32_t* d_tables, int max_blocks, const int32_t* d_chunks,
                           const int32_t* d_tile_map, int n_tiles, int n_groups, int max_pieces,
                           void* out, int out_stride, int n_q_heads, void* workspace,
                           size_t workspace_bytes, af_stream_t stream) {
    const bool pieced = max_pieces > 0;  // a 4-int piece map
    if (!q || !pool || !pool->base || !d_tables || !d_chunks || !d_tile_map || !out ||
        n_tiles < 0 || n_q_heads <= 0 || max_blocks <= 0)
        return AF_ERR_INVALID_ARG;
    if (pieced && (max_pieces > kPfMaxPieces || n_groups < 0 ||
                   int64_t(n_groups) * n_q_heads > kMaxCounters))
        return AF_ERR_INVALID_ARG;
    if (layer < 0 || layer >= pool->n_layers || pool->n_kv_heads <= 0 ||
        n_q_heads % pool->n_kv_heads || pool->total_blocks <= 0 ||
        (pool->flags & ~AF_KV_POOL_SHARED_BLOCKS))
        return AF_ERR_INVALID_ARG;
    const bool fp8 = pool->dtype == AF_KV_FP8_E4M3;
    if ((!fp8 && pool->dtype != AF_KV_FP16) || pool->head_dim != kPfHd) return AF_ERR_UNSUPPORTED;
    if (fp8 && !pool->scales) return AF_ERR_INVALID_ARG;
    const int bs = pool->block_size;
    if (bs < 8 || (bs & (bs - 1))) return AF_ERR_INVALID_ARG;
    const int q_dim = n_q_heads * kPfHd;
    if (q_stride < q_dim || out_stride < q_dim || q_stride % 8 || out_stride % 8)
        return AF_ERR_INVALID_ARG;
    if (!aligned16(q) || !aligned16(out) || !aligned16(pool->base)) return AF_ERR_INVALID_ARG;
    if (n_tiles == 0) return AF_OK;
    const int64_t kv_stride = int64_t(pool->n_kv_heads) * kPfHd;
    const size_t esz = fp8 ? 1 : 2;
    const size_t slab = size_t(pool->total_blocks) * bs * kv_stride * esz;
    const char* base = static_cast<const char*>(pool->base);
    PrefillArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.q_stride = q_stride;
    a.k = reinterpret_cast<const uint16_t*>(base + size_t(2 * layer) * slab);
    a.v = reinterpret_cast<const uint16_t*>(base + size_t(2 * layer + 1) * slab);
    a.kv_stride = kv_stride;
    a.kv_row_bytes = uint32_t(kv_stride * esz);
    a.scales = fp8 ? pool->scales + size_t(layer) * 2 * pool->n_kv_heads : nullptr;
    a.out = static_cast<uint16_t*>(out);
    a.out_stride = out_stride;
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = pool->n_kv_heads;
    a.scale_log2 = float(1.4426950408889634 / std::sqrt(double(kPfHd)));
    a.table = d_tables;
    a.bs_log2 = __builtin_ctz(unsigned(bs));
    a.max_block = int32_t(std::min<int64_t>(pool->total_blocks - 1, INT32_MAX));
    a.tile_map = d_tile_map;
    a.chunks = d_chunks;
    a.max_blocks = max_blocks;
    if (pieced) {
        a.piece_map = 1;
        a.n_pieces = max_pieces;
        if (max_pieces > 1) {
            if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u) ||
                workspace_bytes < record_workspace_bytes(n_groups, n_q_heads, max_pieces))
                return AF_ERR_WORKSPACE;
            carve_records(a, workspace, n_groups, max_pieces);
        }
    }
    const dim3 grid(n_tiles * n_q_heads), block(kPfThreads);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (fp8)
        hipLaunchKernelGGL((prefill_attention_kernel<true, true>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((prefill_attention_kernel<true, false>), grid, block, 0, s, a);
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" int af_paged_prefill_attention_batched(
    const void* q, int q_stride, const af_kv_pool* pool, int layer, const int32_t* d_tables,
    int max_blocks, const int32_t* d_chunks, const int32_t* d_tile_map, int n_tiles, void* out,
    int out_stride, int n_q_heads, af_stream_t stream) {
    return prefill_batched(q, q_stride, pool, layer, d_tables, max_blocks, d_chunks, d_tile_map,
                           n_tiles, 0, 0, out, out_stride, n_q_heads, nullptr, 0, stream);
}

extern "C" int af_paged_prefill_attention_batched_ws(
    const void* q, int q_stride, const af_kv_pool* pool, int layer, const int32_t* d_tables,
    int max_blocks, const int32_t* d_chunks, const int32_t* d_piece_map, int n_entries,
    int n_groups, int max_pieces, void* out, int out_stride, int n_q_heads, void* workspace,
    size_t workspace_bytes, af_stream_t stream) {
    if (max_pieces < 1) return AF_ERR_INVALID_ARG;
    return prefill_batched(q, q_stride, pool, layer, d_tables, max_blocks, d_chunks, d_piece_map,
                           n_entries, n_groups, max_pieces, out, out_stride, n_q_heads, workspace,
                           workspace_bytes, stream);
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
