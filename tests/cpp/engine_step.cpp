// engine_step.cpp — a C++ host that drives one decode step through the C++
// operator and memory API (include/ops/kernel.h, include/memory/block_manager.h,
// include/server/scheduler.h) the way the reference engine calls its launchers
// (src/core/engine.cu:326-370: launch_rope, launch_write_kv_cache,
// launch_cached_attention on one stream), then the paged step of the server
// sandbox (BlockManager fork + copy-on-write, paged append, paged attention,
// and the shared-prefix form over the forked pair), and a decode step of
// several layers over the engine's one-arena KV pool [L0_K | L0_V | L1_K | ...]
// (engine.cu:187-215, model_state.h:56-64), and a prompt chunk's causal
// attention through the key-piece launcher (launch_prefill_attention_ws).
// Inputs come from a fixed xorshift stream; inputs and outputs are written to
// <out_dir>/*.bin so tests/test_gpu_cpp_host.py can check them against the
// oracle. Exit status 0 only if every call succeeded and the in-program checks
// held (the fused launch equals the three-launch sequence bit for bit).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "memory/alloc.h"
#include "memory/block_manager.h"
#include "ops/kernel.h"

namespace {

constexpr int NH = 24, NKV = 8, HD = 128;
constexpr int Q_DIM = NH * HD, KV_DIM = NKV * HD, QKV = Q_DIM + 2 * KV_DIM;
constexpr int MAX_SEQ = 1024;
constexpr float THETA = 500000.0f;

#define HIP_OK(x)                                                                        \
    do {                                                                                 \
        hipError_t e_ = (x);                                                             \
        if (e_ != hipSuccess)                                                            \
            throw std::runtime_error(std::string(#x) + ": " + hipGetErrorString(e_));   \
    } while (0)

// xorshift64* -> uniform [-2, 2) rounded to fp16 bits (round to nearest even).
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
    uint64_t next() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return s * 0x2545F4914F6CDD1Dull;
    }
    uint16_t half_bits() {
        const float f = float(int64_t(next() >> 11) - (int64_t(1) << 52)) * 0x1p-51f;
        return __half_as_ushort(__float2half_rn(f));
    }
};

std::vector<uint16_t> randn_like(size_t n, uint64_t seed) {
    Rng r(seed);
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = r.half_bits();
    return v;
}

void save(const std::string& dir, const char* name, const void* p, size_t bytes) {
    const std::string path = dir + "/" + name + ".bin";
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(p, 1, bytes, f) != bytes) throw std::runtime_error("write " + path);
    std::fclose(f);
}

template <typename T>
T* dev_upload(const std::vector<T>& h) {
    T* d = nullptr;
    HIP_OK(hipMalloc(&d, h.size() * sizeof(T)));
    HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

template <typename T>
std::vector<T> dev_download(const T* d, size_t n) {
    std::vector<T> h(n);
    HIP_OK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

// The reference's decode step for one layer at position pos, three launches,
// and the fused launch on a copy of the same inputs.
int contiguous_step(const std::string& dir, hipStream_t s) {
    const int pos = 300;
    auto qkv = randn_like(QKV, 1);
    auto kc = randn_like(size_t(MAX_SEQ) * KV_DIM, 2);
    auto vc = randn_like(size_t(MAX_SEQ) * KV_DIM, 3);
    save(dir, "c_qkv_in", qkv.data(), qkv.size() * 2);
    save(dir, "c_k_in", kc.data(), kc.size() * 2);
    save(dir, "c_v_in", vc.data(), vc.size() * 2);

    float *d_cos = nullptr, *d_sin = nullptr;
    HIP_OK(hipMalloc(&d_cos, size_t(MAX_SEQ) * HD / 2 * 4));
    HIP_OK(hipMalloc(&d_sin, size_t(MAX_SEQ) * HD / 2 * 4));
    build_rope_cache(d_cos, d_sin, MAX_SEQ, HD, THETA, s);

    uint16_t* d_qkv = dev_upload(qkv);
    uint16_t* d_k = dev_upload(kc);
    uint16_t* d_v = dev_upload(vc);
    uint16_t* d_qkv2 = dev_upload(qkv);
    uint16_t* d_k2 = dev_upload(kc);
    uint16_t* d_v2 = dev_upload(vc);
    uint16_t *d_out = nullptr, *d_out2 = nullptr;
    HIP_OK(hipMalloc(&d_out, Q_DIM * 2));
    HIP_OK(hipMalloc(&d_out2, Q_DIM * 2));

    // engine.cu:326-370
    View q = create_contiguous_view(d_qkv, DataType::FP16, {1, Q_DIM});
    View k = create_contiguous_view(d_qkv + Q_DIM, DataType::FP16, {1, KV_DIM});
    View qkv_v = create_contiguous_view(d_qkv, DataType::FP16, {1, QKV});
    View k_cache = create_contiguous_view(d_k, DataType::FP16, {MAX_SEQ, KV_DIM});
    View v_cache = create_contiguous_view(d_v, DataType::FP16, {MAX_SEQ, KV_DIM});
    launch_rope(q, k, d_cos + size_t(pos) * (HD / 2), d_sin + size_t(pos) * (HD / 2), 1, NKV, NH,
                HD, s);
    launch_write_kv_cache(qkv_v, k_cache, v_cache, pos, Q_DIM, KV_DIM, s);
    launch_cached_attention(reinterpret_cast<const __half*>(d_qkv),
                            reinterpret_cast<const __half*>(d_k),
                            reinterpret_cast<const __half*>(d_v),
                            reinterpret_cast<__half*>(d_out), pos + 1, HD, NH, NKV, s);

    // the same step with the fused append
    View qkv2 = create_contiguous_view(d_qkv2, DataType::FP16, {1, QKV});
    View k2 = create_contiguous_view(d_k2, DataType::FP16, {MAX_SEQ, KV_DIM});
    View v2 = create_contiguous_view(d_v2, DataType::FP16, {MAX_SEQ, KV_DIM});
    launch_rope_append(qkv2, k2, v2, d_cos, d_sin, pos, nullptr, NH, NKV, HD, s);
    launch_cached_attention(reinterpret_cast<const __half*>(d_qkv2),
                            reinterpret_cast<const __half*>(d_k2),
                            reinterpret_cast<const __half*>(d_v2),
                            reinterpret_cast<__half*>(d_out2), pos + 1, HD, NH, NKV, s);
    HIP_OK(hipStreamSynchronize(s));

    auto qkv_after = dev_download(d_qkv, QKV);
    auto k_after = dev_download(d_k, size_t(MAX_SEQ) * KV_DIM);
    auto v_after = dev_download(d_v, size_t(MAX_SEQ) * KV_DIM);
    auto out = dev_download(d_out, Q_DIM);
    save(dir, "c_qkv_out", qkv_after.data(), qkv_after.size() * 2);
    save(dir, "c_k_out", k_after.data(), k_after.size() * 2);
    save(dir, "c_v_out", v_after.data(), v_after.size() * 2);
    save(dir, "c_attn", out.data(), out.size() * 2);
    int bad = 0;
    if (dev_download(d_qkv2, QKV) != qkv_after) bad |= 1;
    if (dev_download(d_k2, size_t(MAX_SEQ) * KV_DIM) != k_after) bad |= 2;
    if (dev_download(d_v2, size_t(MAX_SEQ) * KV_DIM) != v_after) bad |= 4;
    if (dev_download(d_out2, Q_DIM) != out) bad |= 8;
    for (void* p : {(void*)d_cos, (void*)d_sin, (void*)d_qkv, (void*)d_k, (void*)d_v,
                    (void*)d_qkv2, (void*)d_k2, (void*)d_v2, (void*)d_out, (void*)d_out2})
        HIP_OK(hipFree(p));
    if (bad) std::fprintf(stderr, "fused step differs from the three-launch step (mask %d)\n", bad);
    return bad;
}

// The paged step: two sequences, a fork of the first (shared partial tail),
// one decode token each; the fork's append is a copy-on-write.
int paged_step(const std::string& dir, hipStream_t s) {
    using atomflow::server::AppendSlot;
    using atomflow::server::BlockManager;
    using atomflow::server::PoolConfig;
    const int bs = 16, total = 64, max_pos = 512;
    BlockManager bm;
    PoolConfig cfg;
    cfg.total_blocks = total;
    cfg.block_size = bs;
    cfg.n_layers = 1;
    cfg.n_kv_heads = NKV;
    cfg.head_dim = HD;
    bm.initialize(cfg, /*allocate_pool=*/true);
    const af_kv_pool pool = bm.pool_desc();
    const size_t pool_halves = size_t(2) * total * bs * KV_DIM;
    auto pool_init = randn_like(pool_halves, 4);
    HIP_OK(hipMemcpy(pool.base, pool_init.data(), pool_halves * 2, hipMemcpyHostToDevice));

    const int lens[2] = {100, 37};
    int seqs[3];
    for (int i = 0; i < 2; ++i) {
        seqs[i] = bm.create_sequence();
        int first = 0;
        if (bm.extend(seqs[i], lens[i], &first, nullptr) != AF_OK) return 16;
    }
    seqs[2] = bm.fork_sequence(seqs[0]);  // shares seq 0's blocks, tail has 4 rows
    AppendSlot slots[3];
    if (bm.plan_decode(seqs, 3, slots) != AF_OK) return 17;
    std::vector<int32_t> copies;
    for (const AppendSlot& a : slots)
        if (a.cow.src >= 0) copies.insert(copies.end(), {a.cow.src, a.cow.dst, a.cow.rows});
    if (copies.size() != 3) return 18;  // exactly one copy-on-write (the fork or its parent)

    const int max_blocks = (max_pos + bs - 1) / bs;
    std::vector<int32_t> tables(size_t(3) * max_blocks, 0), seq_lens(3);
    std::vector<int64_t> slot_v(3);
    std::vector<int32_t> pos_v(3);
    for (int b = 0; b < 3; ++b) {
        const auto& t = bm.table(seqs[b]);
        for (size_t j = 0; j < t.block_ids.size(); ++j) tables[size_t(b) * max_blocks + j] = t.block_ids[j];
        seq_lens[size_t(b)] = bm.seq_len(seqs[b]);
        slot_v[size_t(b)] = slots[b].slot;
        pos_v[size_t(b)] = slots[b].position;
    }
    auto qkv = randn_like(size_t(3) * QKV, 5);
    save(dir, "p_qkv_in", qkv.data(), qkv.size() * 2);
    save(dir, "p_pool_in", pool_init.data(), pool_halves * 2);
    save(dir, "p_tables", tables.data(), tables.size() * 4);
    save(dir, "p_lens", seq_lens.data(), seq_lens.size() * 4);
    save(dir, "p_slots", slot_v.data(), slot_v.size() * 8);
    save(dir, "p_positions", pos_v.data(), pos_v.size() * 4);
    save(dir, "p_copies", copies.data(), copies.size() * 4);

    float *d_cos = nullptr, *d_sin = nullptr;
    HIP_OK(hipMalloc(&d_cos, size_t(max_pos) * HD / 2 * 4));
    HIP_OK(hipMalloc(&d_sin, size_t(max_pos) * HD / 2 * 4));
    build_rope_cache(d_cos, d_sin, max_pos, HD, THETA, s);
    uint16_t* d_qkv = dev_upload(qkv);
    int32_t* d_tables = dev_upload(tables);
    int32_t* d_lens = dev_upload(seq_lens);
    int64_t* d_slots = dev_upload(slot_v);
    int32_t* d_pos = dev_upload(pos_v);
    int32_t* d_copies = dev_upload(copies);
    const std::vector<int32_t> n_copies = {int32_t(copies.size() / 3)};
    int32_t* d_ncopies = dev_upload(n_copies);
    uint16_t* d_out = nullptr;
    HIP_OK(hipMalloc(&d_out, size_t(3) * Q_DIM * 2));
    const size_t ws_bytes = af_attention_workspace_size(3, NH, NKV, HD, 0);
    void* ws = nullptr;
    HIP_OK(hipMalloc(&ws, ws_bytes));
    if (af_attention_workspace_init(ws, ws_bytes, s) != AF_OK) return 19;

    launch_kv_copy_blocks(pool, d_copies, d_ncopies, 3, s);
    launch_paged_rope_append(reinterpret_cast<__half*>(d_qkv), 3, pool, 0, d_slots, d_pos, d_cos,
                             d_sin, max_pos, NH, s);
    int max_len = 0;
    for (int l : seq_lens) max_len = l > max_len ? l : max_len;
    launch_paged_attention(reinterpret_cast<const __half*>(d_qkv), QKV, pool, 0, d_tables,
                           max_blocks, d_lens, 3, max_len, reinterpret_cast<__half*>(d_out), Q_DIM,
                           NH, 0, ws, ws_bytes, s);
    // Seq 2 is a fork of seq 0: their rows [0, 100) hold the same values (the
    // shared partial tail was copied above). The shared-prefix form over
    // {seq 0, seq 2} (q rows 0 and 2 of qkv_out: stride 2 * QKV) must agree with
    // the paged attention of those rows within twice the attention tolerance.
    std::vector<int32_t> t02(size_t(2) * max_blocks), l02 = {seq_lens[0], seq_lens[2]};
    std::memcpy(t02.data(), tables.data(), size_t(max_blocks) * 4);
    std::memcpy(t02.data() + max_blocks, tables.data() + size_t(2) * max_blocks,
                size_t(max_blocks) * 4);
    int32_t* d_t02 = dev_upload(t02);
    int32_t* d_l02 = dev_upload(l02);
    uint16_t* d_out_sp = nullptr;
    HIP_OK(hipMalloc(&d_out_sp, size_t(2) * Q_DIM * 2));
    launch_paged_attention_shared_prefix(reinterpret_cast<const __half*>(d_qkv), 2 * QKV, pool, 0,
                                         d_t02, lens[0], 0, d_t02, max_blocks, d_l02, 2, max_len,
                                         reinterpret_cast<__half*>(d_out_sp), Q_DIM, NH, 0, ws,
                                         ws_bytes, s);
    HIP_OK(hipStreamSynchronize(s));
    auto pool_out = dev_download(static_cast<const uint16_t*>(pool.base), pool_halves);
    auto qkv_out = dev_download(d_qkv, size_t(3) * QKV);
    auto out = dev_download(d_out, size_t(3) * Q_DIM);
    auto out_sp = dev_download(d_out_sp, size_t(2) * Q_DIM);
    for (int r = 0; r < 2; ++r)
        for (int e = 0; e < Q_DIM; ++e) {
            const float a = __half2float(__ushort_as_half(out_sp[size_t(r) * Q_DIM + e]));
            const float b = __half2float(__ushort_as_half(out[size_t(2 * r) * Q_DIM + e]));
            if (!(std::fabs(a - b) <= 4e-3f + 2e-2f * std::fabs(b))) return 20;
        }
    HIP_OK(hipFree(d_t02));
    HIP_OK(hipFree(d_l02));
    HIP_OK(hipFree(d_out_sp));
    save(dir, "p_pool_out", pool_out.data(), pool_out.size() * 2);
    save(dir, "p_qkv_out", qkv_out.data(), qkv_out.size() * 2);
    save(dir, "p_attn", out.data(), out.size() * 2);
    for (void* p : {(void*)d_cos, (void*)d_sin, (void*)d_qkv, (void*)d_tables, (void*)d_lens,
                    (void*)d_slots, (void*)d_pos, (void*)d_copies, (void*)d_ncopies,
                    (void*)d_out, ws})
        HIP_OK(hipFree(p));
    return 0;
}

// The engine's KV pool: one ArenaAllocator, [L0_K | L0_V | L1_K | ...], each
// slab MAX_SEQ x KV_DIM fp16 wrapped in a View (engine.cu:187-215). Rows
// [pos, MAX_SEQ) of every slab hold NaN, so a read outside a layer's own rows
// [0, pos) (or past the end of the slab below it) poisons that layer's output.
// Every layer runs the one-launch step (af_decode_attention_fused) on this
// pool and the reference's three launches on a second pool; the two must
// agree bit for bit, and the test compares the whole first pool with the
// oracle, so a write outside the layer's row `pos` shows up too.
int pooled_step(const std::string& dir, hipStream_t s) {
    constexpr int NL = 4;
    const int pos = 700;
    const size_t slab = size_t(MAX_SEQ) * KV_DIM * 2;
    ArenaAllocator arena(NL * 2 * slab);
    ArenaAllocator arena2(NL * 2 * slab);
    View kc[NL], vc[NL], kc2[NL], vc2[NL];
    for (int l = 0; l < NL; ++l) {
        kc[l] = create_contiguous_view(arena.allocate(slab), DataType::FP16, {MAX_SEQ, KV_DIM});
        vc[l] = create_contiguous_view(arena.allocate(slab), DataType::FP16, {MAX_SEQ, KV_DIM});
        kc2[l] = create_contiguous_view(arena2.allocate(slab), DataType::FP16, {MAX_SEQ, KV_DIM});
        vc2[l] = create_contiguous_view(arena2.allocate(slab), DataType::FP16, {MAX_SEQ, KV_DIM});
        char* base = static_cast<char*>(arena.base());
        if (kc[l].data_ptr != base + (2 * l) * slab || vc[l].data_ptr != base + (2 * l + 1) * slab)
            return 40;
    }
    const size_t halves = size_t(NL) * 2 * MAX_SEQ * KV_DIM;
    std::vector<uint16_t> pool(halves);
    for (int sl = 0; sl < 2 * NL; ++sl) {
        auto rows = randn_like(size_t(pos) * KV_DIM, 60 + sl);
        uint16_t* dst = pool.data() + size_t(sl) * MAX_SEQ * KV_DIM;
        std::memcpy(dst, rows.data(), rows.size() * 2);
        for (size_t i = size_t(pos) * KV_DIM; i < size_t(MAX_SEQ) * KV_DIM; ++i) dst[i] = 0x7e00;
    }
    auto qkv = randn_like(size_t(NL) * QKV, 70);
    save(dir, "pl_pool_in", pool.data(), halves * 2);
    save(dir, "pl_qkv_in", qkv.data(), qkv.size() * 2);
    HIP_OK(hipMemcpy(arena.base(), pool.data(), halves * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(arena2.base(), pool.data(), halves * 2, hipMemcpyHostToDevice));
    float *d_cos = nullptr, *d_sin = nullptr;
    HIP_OK(hipMalloc(&d_cos, size_t(MAX_SEQ) * HD / 2 * 4));
    HIP_OK(hipMalloc(&d_sin, size_t(MAX_SEQ) * HD / 2 * 4));
    build_rope_cache(d_cos, d_sin, MAX_SEQ, HD, THETA, s);
    uint16_t* d_qkv = dev_upload(qkv);
    uint16_t* d_qkv2 = dev_upload(qkv);
    uint16_t *d_out = nullptr, *d_out2 = nullptr;
    HIP_OK(hipMalloc(&d_out, size_t(NL) * Q_DIM * 2));
    HIP_OK(hipMalloc(&d_out2, size_t(NL) * Q_DIM * 2));
    const size_t ws_bytes = af_attention_workspace_size(1, NH, NKV, HD, 0);
    void* ws = nullptr;
    HIP_OK(hipMalloc(&ws, ws_bytes));
    if (af_attention_workspace_init(ws, ws_bytes, s) != AF_OK) return 41;
    // the split count launch_cached_attention picks for pos + 1 rows
    const int splits = af_attention_default_splits(pos + 1, 1, NKV);
    for (int l = 0; l < NL; ++l) {
        uint16_t* q = d_qkv + size_t(l) * QKV;
        if (af_decode_attention_fused(q, kc[l].data_ptr, vc[l].data_ptr, d_cos, d_sin, pos,
                                      nullptr, MAX_SEQ, d_out + size_t(l) * Q_DIM, NH, NKV, HD,
                                      splits, ws, ws_bytes, nullptr, s) != AF_OK)
            return 42;
        // the reference's three launches on the second pool (engine.cu:340-369)
        uint16_t* q2 = d_qkv2 + size_t(l) * QKV;
        View qv = create_contiguous_view(q2, DataType::FP16, {1, Q_DIM});
        View kv = create_contiguous_view(q2 + Q_DIM, DataType::FP16, {1, KV_DIM});
        View qkv_v = create_contiguous_view(q2, DataType::FP16, {1, QKV});
        launch_rope(qv, kv, d_cos + size_t(pos) * (HD / 2), d_sin + size_t(pos) * (HD / 2), 1, NKV,
                    NH, HD, s);
        launch_write_kv_cache(qkv_v, kc2[l], vc2[l], pos, Q_DIM, KV_DIM, s);
        launch_cached_attention(reinterpret_cast<const __half*>(q2),
                                static_cast<const __half*>(kc2[l].data_ptr),
                                static_cast<const __half*>(vc2[l].data_ptr),
                                reinterpret_cast<__half*>(d_out2 + size_t(l) * Q_DIM), pos + 1, HD,
                                NH, NKV, s);
    }
    HIP_OK(hipStreamSynchronize(s));
    auto pool_out = dev_download(static_cast<const uint16_t*>(arena.base()), halves);
    auto qkv_out = dev_download(d_qkv, size_t(NL) * QKV);
    auto out = dev_download(d_out, size_t(NL) * Q_DIM);
    save(dir, "pl_pool_out", pool_out.data(), halves * 2);
    save(dir, "pl_qkv_out", qkv_out.data(), qkv_out.size() * 2);
    save(dir, "pl_attn", out.data(), out.size() * 2);
    int bad = 0;
    if (dev_download(static_cast<const uint16_t*>(arena2.base()), halves) != pool_out) bad |= 1;
    if (dev_download(d_qkv2, size_t(NL) * QKV) != qkv_out) bad |= 2;
    // Same split count on both sides, so the attention bits agree.
    if (dev_download(d_out2, size_t(NL) * Q_DIM) != out) bad |= 4;
    for (void* p : {(void*)d_cos, (void*)d_sin, (void*)d_qkv, (void*)d_qkv2, (void*)d_out,
                    (void*)d_out2, ws})
        HIP_OK(hipFree(p));
    if (bad) std::fprintf(stderr, "pooled fused step differs from the three launches (mask %d)\n", bad);
    return bad ? 43 : 0;
}

}  // namespace

// A 300-token prompt chunk at p0 700 (kv_len 1000) through
// launch_prefill_attention_ws with the library's choice of key pieces (its three
// query tiles are cut), and the same chunk through launch_prefill_attention.
int prefill_step(const std::string& dir, hipStream_t s) {
    const int p0 = 700, n = 300, kv_len = 1000;
    auto q = randn_like(size_t(n) * Q_DIM, 31);
    auto kc = randn_like(size_t(MAX_SEQ) * KV_DIM, 32);
    auto vc = randn_like(size_t(MAX_SEQ) * KV_DIM, 33);
    save(dir, "f_q", q.data(), q.size() * 2);
    save(dir, "f_k", kc.data(), kc.size() * 2);
    save(dir, "f_v", vc.data(), vc.size() * 2);
    uint16_t* d_q = dev_upload(q);
    uint16_t* d_k = dev_upload(kc);
    uint16_t* d_v = dev_upload(vc);
    uint16_t *d_out = nullptr, *d_plain = nullptr;
    HIP_OK(hipMalloc(&d_out, size_t(n) * Q_DIM * 2));
    HIP_OK(hipMalloc(&d_plain, size_t(n) * Q_DIM * 2));
    const size_t ws_bytes = af_prefill_workspace_size(p0, n, kv_len, NH, 0);
    void* ws = nullptr;
    HIP_OK(hipMalloc(&ws, ws_bytes));
    if (af_attention_workspace_init(ws, ws_bytes, s) != AF_OK) throw std::runtime_error("ws init");
    View k_cache = create_contiguous_view(d_k, DataType::FP16, {MAX_SEQ, KV_DIM});
    View v_cache = create_contiguous_view(d_v, DataType::FP16, {MAX_SEQ, KV_DIM});
    const __half* hq = reinterpret_cast<const __half*>(d_q);
    launch_prefill_attention_ws(hq, Q_DIM, k_cache, v_cache, reinterpret_cast<__half*>(d_out),
                                Q_DIM, p0, n, kv_len, NH, NKV, HD, 0, ws, ws_bytes, s);
    launch_prefill_attention(hq, Q_DIM, k_cache, v_cache, reinterpret_cast<__half*>(d_plain),
                             Q_DIM, p0, n, kv_len, NH, NKV, HD, s);
    HIP_OK(hipStreamSynchronize(s));
    auto out = dev_download(d_out, size_t(n) * Q_DIM);
    auto plain = dev_download(d_plain, size_t(n) * Q_DIM);
    save(dir, "f_attn", out.data(), out.size() * 2);
    save(dir, "f_attn_plain", plain.data(), plain.size() * 2);
    const uint64_t ws_size = ws_bytes;
    save(dir, "f_ws_bytes", &ws_size, sizeof(ws_size));
    for (void* p : {(void*)d_q, (void*)d_k, (void*)d_v, (void*)d_out, (void*)d_plain, ws})
        HIP_OK(hipFree(p));
    return 0;
}

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s OUT_DIR\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    try {
        HIP_OK(hipSetDevice(0));
        hipStream_t s = nullptr;
        HIP_OK(hipStreamCreate(&s));
        int rc = contiguous_step(dir, s);
        if (rc == 0) rc = paged_step(dir, s);
        if (rc == 0) rc = pooled_step(dir, s);
        if (rc == 0) rc = prefill_step(dir, s);
        HIP_OK(hipStreamDestroy(s));
        if (rc == 0) std::puts("ok");
        return rc;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 3;
    }
}
