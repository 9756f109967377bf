// memory_api.cpp — CPU checks of the memory API kept from the reference:
//  * ArenaAllocator (include/memory/alloc.h:17-29): 128-B bump allocation, the
//    out-of-memory throw that leaves the arena unchanged, reset_workspace;
//  * MemoryPlanner (include/memory/memory_planner.h:11-26): 16-B typed bump
//    allocation and its "Arena Out Of Memory!" throw;
//  * the engine's KV pool carve (src/core/engine.cu:187-215,
//    include/core/model_state.h:56-64): one arena, [L0_K | L0_V | L1_K | ...],
//    MAX_SEQ_LEN x KV_DIM fp16 slabs wrapped in Views whose 64-bit dims and
//    strides address past 2^31 elements.
// The pool carve uses a borrowed arena at a device-like address that is never
// dereferenced, so no GPU is needed. Prints "ok" and exits 0 when every check
// holds; otherwise prints the first failed check and exits 1.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>

#include "core/view.h"
#include "memory/alloc.h"
#include "memory/memory_planner.h"

#define CHECK(c)                                                   \
    do {                                                           \
        if (!(c)) {                                                \
            std::printf("FAIL line %d: %s\n", __LINE__, #c);       \
            return 1;                                              \
        }                                                          \
    } while (0)

namespace {

int arena_checks() {
    alignas(128) static unsigned char buf[4096];
    ArenaAllocator a(buf, 1000);
    CHECK(a.get_capacity() == 1000 && a.get_offset() == 0 && a.base() == buf);
    unsigned char* p0 = static_cast<unsigned char*>(a.allocate(1));
    unsigned char* p1 = static_cast<unsigned char*>(a.allocate(128));
    unsigned char* p2 = static_cast<unsigned char*>(a.allocate(129));
    CHECK(p0 == buf && p1 == buf + 128 && p2 == buf + 256);  // 1 -> 128, 128 -> 128, 129 -> 256
    CHECK(a.get_offset() == 512);
    for (unsigned char* p : {p0, p1, p2}) CHECK((reinterpret_cast<uintptr_t>(p) & 127) == 0);
    CHECK(a.allocate(384) == buf + 512 && a.get_offset() == 896);
    bool threw = false;
    try {
        (void)a.allocate(1);  // 896 + 128 > 1000
    } catch (const std::runtime_error& e) {
        threw = std::strstr(e.what(), "out of memory") != nullptr;
    }
    CHECK(threw && a.get_offset() == 896);  // a failed allocation changes nothing
    a.reset_workspace(128);
    CHECK(a.allocate(200) == buf + 128 && a.get_offset() == 384);
    threw = false;
    try {
        ArenaAllocator b(buf + 8, 100);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    CHECK(threw);
    // The owning form: one hipMalloc rounded up to 128 B, or a runtime_error
    // naming the failed allocation (no device in the build container).
    try {
        ArenaAllocator o(1000);
        CHECK(o.get_capacity() == 1024 && (reinterpret_cast<uintptr_t>(o.base()) & 127) == 0);
        CHECK(o.allocate(1000) == o.base() && o.get_offset() == 1024);
        std::printf("owning arena: allocated %zu B\n", o.get_capacity());
    } catch (const std::runtime_error& e) {
        CHECK(std::strstr(e.what(), "failed to allocate") != nullptr);
        std::printf("owning arena: %s\n", e.what());
    }
    return 0;
}

int planner_checks() {
    alignas(16) static unsigned char buf[256];
    MemoryPlanner m(buf, 100);
    float* f = m.allocate<float>(3);  // 12 B -> 16
    CHECK(reinterpret_cast<unsigned char*>(f) == buf && m.get_offset() == 16);
    uint8_t* u = m.allocate<uint8_t>(1);  // 1 B -> 16
    CHECK(u == buf + 16 && m.get_offset() == 32);
    double* d = m.allocate<double>(8);  // 64 B
    CHECK(reinterpret_cast<unsigned char*>(d) == buf + 32 && m.get_offset() == 96);
    bool threw = false;
    try {
        (void)m.allocate<uint8_t>(5);  // 96 + 16 > 100
    } catch (const std::runtime_error& e) {
        threw = std::strcmp(e.what(), "Arena Out Of Memory!") == 0;
    }
    CHECK(threw && m.get_offset() == 96);
    m.reset_to(16);
    CHECK(m.allocate<uint16_t>(8) == reinterpret_cast<uint16_t*>(buf + 16));
    return 0;
}

int kv_pool_checks() {
    // Llama-3.2-3B (28 layers, KV_DIM 1024) at MAX_SEQ_LEN 131072: 56 slabs of
    // 256 MiB, 14 GiB in all, carved in the engine's order.
    constexpr int NL = 28;
    constexpr int64_t MAX_SEQ = 131072, KV_DIM = 1024;
    const size_t slab = size_t(MAX_SEQ) * KV_DIM * 2;
    void* fake = reinterpret_cast<void*>(uintptr_t(0x7f0000000000ull));
    unsigned char* base = static_cast<unsigned char*>(fake);
    ArenaAllocator pool(fake, NL * 2 * slab);
    View k[NL], v[NL];
    for (int l = 0; l < NL; ++l) {
        k[l] = create_contiguous_view(pool.allocate(slab), DataType::FP16, {MAX_SEQ, KV_DIM});
        v[l] = create_contiguous_view(pool.allocate(slab), DataType::FP16, {MAX_SEQ, KV_DIM});
        CHECK(k[l].data_ptr == base + size_t(2 * l) * slab);
        CHECK(v[l].data_ptr == base + size_t(2 * l + 1) * slab);
        CHECK(k[l].num_dims == 2 && k[l].dims[0] == MAX_SEQ && k[l].dims[1] == KV_DIM);
        CHECK(k[l].strides[0] == KV_DIM && k[l].strides[1] == 1);
        CHECK(k[l].numel() == MAX_SEQ * KV_DIM && v[l].dtype == DataType::FP16);
    }
    CHECK(pool.get_offset() == NL * 2 * slab);
    // The last element of the pool, from the pool base: 7.5e9 elements, past
    // the 2^31 limit of the reference's int32 View arithmetic.
    const size_t last = size_t(static_cast<unsigned char*>(v[NL - 1].data_ptr) - base) / 2 +
                        v[NL - 1].offset(MAX_SEQ - 1, KV_DIM - 1);
    CHECK(last == size_t(NL) * 2 * MAX_SEQ * KV_DIM - 1 && last > (size_t(1) << 31));
    // A paged FP8 pool of BASELINE configs[4]'s size as one View.
    const int64_t rows = int64_t(NL) * 2 * 54582 * 32;
    View big = create_contiguous_view(fake, DataType::FP8_E4M3, {rows, KV_DIM});
    CHECK(big.numel() == rows * KV_DIM && big.numel() > (int64_t(1) << 36));
    CHECK(big.offset(rows - 1, KV_DIM - 1) == size_t(big.numel() - 1));
    CHECK(dtype_size(DataType::FP32) == 4 && dtype_size(DataType::FP16) == 2 &&
          dtype_size(DataType::BF16) == 2 && dtype_size(DataType::FP8_E4M3) == 1);
    return 0;
}

}  // namespace

int main() {
    if (arena_checks() || planner_checks() || kv_pool_checks()) return 1;
    std::puts("ok");
    return 0;
}
