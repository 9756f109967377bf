// kv_blocks.hip — paged-pool data movement for gfx950: block-table gather,
// copy-on-write block copies, FP8 quantisation, and fill / synthetic-data
// kernels. All copies move 16-B vectors; HBM-bound.
#include <cmath>

#include "af_common.h"
#include "af_device.h"

namespace af {
namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__global__ void fill_u32_kernel(uint32_t* __restrict__ dst, uint32_t value, size_t n) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = value;
}

// Gather of logical rows [0, seq_len) of one layer slab into a contiguous
// buffer: row t comes from block table[t / bs] at offset t % bs. One 16-B
// vector per thread; block ids are clamped into the pool.
__global__ void paged_gather_kernel(const uint8_t* __restrict__ k_slab,
                                    const uint8_t* __restrict__ v_slab,
                                    const int32_t* __restrict__ table, int seq_len, int block_shift,
                                    int64_t total_blocks, int row_vecs, uint8_t* __restrict__ k_dst,
                                    uint8_t* __restrict__ v_dst) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= int64_t(seq_len) * row_vecs) return;
    const int t = int(i / row_vecs);
    const int c = int(i % row_vecs);
    int64_t blk = table[t >> block_shift];
    blk = blk < 0 ? 0 : (blk >= total_blocks ? total_blocks - 1 : blk);
    const int64_t phys = (blk << block_shift) | (t & ((1 << block_shift) - 1));
    const int64_t src = (phys * row_vecs + c) * 16;
    const int64_t dst = i * 16;
    *reinterpret_cast<uint4*>(k_dst + dst) = *reinterpret_cast<const uint4*>(k_slab + src);
    *reinterpret_cast<uint4*>(v_dst + dst) = *reinterpret_cast<const uint4*>(v_slab + src);
}

// Copy-on-write: blockIdx.x = copy index, blockIdx.y = slab (2 * layer + {K,V}).
// Copies rows [0, rows) of block src to block dst. Entries with an id outside
// the pool or rows outside [0, block_size] are skipped.
__global__ void copy_blocks_kernel(uint8_t* __restrict__ base, size_t slab_bytes,
                                   const int32_t* __restrict__ copies,
                                   const int32_t* __restrict__ count, int max_copies,
                                   int64_t total_blocks, int block_size, int row_vecs) {
    const int i = blockIdx.x;
    const int n = min(*count, max_copies);
    if (i >= n) return;
    const int src = copies[3 * i], dst = copies[3 * i + 1], rows = copies[3 * i + 2];
    if (src < 0 || src >= total_blocks || dst < 0 || dst >= total_blocks || rows <= 0 ||
        rows > block_size)
        return;
    uint8_t* slab = base + size_t(blockIdx.y) * slab_bytes;
    const size_t block_bytes = size_t(block_size) * row_vecs * 16;
    const uint4* s = reinterpret_cast<const uint4*>(slab + size_t(src) * block_bytes);
    uint4* d = reinterpret_cast<uint4*>(slab + size_t(dst) * block_bytes);
    const int vecs = rows * row_vecs;
    for (int v = threadIdx.x; v < vecs; v += blockDim.x) d[v] = s[v];
}

__global__ void add_i32_kernel(int32_t* __restrict__ p, int n, int32_t delta) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] += delta;
}

__global__ void fp8_quantize_kernel(const uint16_t* __restrict__ src, uint8_t* __restrict__ dst,
                                    size_t n, float scale) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = uint8_t(quantize_fp8(src[i], scale));
}

// Counter-based N(0,1): SplitMix64 finaliser of (seed, index) -> two 24-bit
// uniforms -> Box-Muller. Deterministic per element, independent of launch shape.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ float randn_at(uint64_t seed, uint64_t i) {
    const uint64_t r = mix64(seed + (i + 1) * 0x9e3779b97f4a7c15ull);
    const float u1 = (float((r >> 40) & 0xffffffu) + 1.0f) * (1.0f / 16777217.0f);  // (0, 1)
    const float u2 = float((r >> 8) & 0xffffffu) * (1.0f / 16777216.0f);
    return __builtin_sqrtf(-2.0f * __logf(u1)) * __cosf(6.283185307179586f * u2);
}

__global__ void randn_f16_kernel(uint16_t* __restrict__ dst, size_t n, uint64_t seed, float sd) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = f2h(randn_at(seed, i) * sd);
}

__global__ void randn_fp8_kernel(uint8_t* __restrict__ dst, size_t n, uint64_t seed,
                                 float inv_scale) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        float v = randn_at(seed, i) * inv_scale;
        v = fminf(fmaxf(v, -448.0f), 448.0f);
        dst[i] = uint8_t(e4m3_encode(v));
    }
}

int grid_for(size_t n, int threads) {
    const size_t blocks = (n + threads - 1) / threads;
    return int(blocks > 65536 ? 65536 : (blocks == 0 ? 1 : blocks));
}

}  // namespace

int fill_u32(void* dst, uint32_t value, size_t n_words, hipStream_t stream) {
    if (!dst) return AF_ERR_INVALID_ARG;
    if (n_words == 0) return AF_OK;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(n_words, 256)), dim3(256), 0, stream,
                       static_cast<uint32_t*>(dst), value, n_words);
    AF_TRY_LAUNCH();
    return AF_OK;
}

}  // namespace af

using namespace af;

static int pool_check(const af_kv_pool* p) {
    if (!p || !p->base || p->n_layers <= 0 || p->n_kv_heads <= 0 || p->head_dim <= 0 ||
        p->total_blocks <= 0 || p->block_size <= 0)
        return AF_ERR_INVALID_ARG;
    if (p->block_size & (p->block_size - 1)) return AF_ERR_UNSUPPORTED;
    if (p->dtype != AF_KV_FP16 && p->dtype != AF_KV_FP8_E4M3) return AF_ERR_UNSUPPORTED;
    if (p->flags & ~AF_KV_POOL_SHARED_BLOCKS) return AF_ERR_INVALID_ARG;
    const size_t esz = p->dtype == AF_KV_FP8_E4M3 ? 1 : 2;
    if ((size_t(p->n_kv_heads) * p->head_dim * esz) % 16) return AF_ERR_UNSUPPORTED;
    if (!aligned16(p->base)) return AF_ERR_INVALID_ARG;
    return AF_OK;
}

extern "C" int af_paged_gather(const af_kv_pool* pool, int layer, const int32_t* d_block_table,
                               int seq_len, void* k_dst, void* v_dst, af_stream_t stream) {
    if (int st = pool_check(pool)) return st;
    if (layer < 0 || layer >= pool->n_layers || !d_block_table || !k_dst || !v_dst || seq_len < 0)
        return AF_ERR_INVALID_ARG;
    if (!aligned16(k_dst) || !aligned16(v_dst)) return AF_ERR_INVALID_ARG;
    if (seq_len == 0) return AF_OK;
    const size_t esz = pool->dtype == AF_KV_FP8_E4M3 ? 1 : 2;
    const size_t row_bytes = size_t(pool->n_kv_heads) * pool->head_dim * esz;
    const size_t slab = size_t(pool->total_blocks) * pool->block_size * row_bytes;
    const uint8_t* base = static_cast<const uint8_t*>(pool->base);
    const int row_vecs = int(row_bytes / 16);
    const int64_t total = int64_t(seq_len) * row_vecs;
    const int threads = 256;
    const int64_t blocks = (total + threads - 1) / threads;
    if (blocks > INT32_MAX) return AF_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(paged_gather_kernel, dim3(unsigned(blocks)), dim3(threads), 0,
                       static_cast<hipStream_t>(stream), base + size_t(2 * layer) * slab,
                       base + size_t(2 * layer + 1) * slab, d_block_table, seq_len,
                       __builtin_ctz(unsigned(pool->block_size)), int64_t(pool->total_blocks),
                       row_vecs, static_cast<uint8_t*>(k_dst), static_cast<uint8_t*>(v_dst));
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" int af_kv_copy_blocks(const af_kv_pool* pool, const int32_t* d_copies,
                                 const int32_t* d_count, int max_copies, af_stream_t stream) {
    if (int st = pool_check(pool)) return st;
    if (!d_copies || !d_count || max_copies < 0) return AF_ERR_INVALID_ARG;
    if (max_copies == 0) return AF_OK;
    const size_t esz = pool->dtype == AF_KV_FP8_E4M3 ? 1 : 2;
    const size_t row_bytes = size_t(pool->n_kv_heads) * pool->head_dim * esz;
    const size_t slab = size_t(pool->total_blocks) * pool->block_size * row_bytes;
    hipLaunchKernelGGL(copy_blocks_kernel, dim3(max_copies, 2 * pool->n_layers), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<uint8_t*>(pool->base), slab,
                       d_copies, d_count, max_copies, int64_t(pool->total_blocks),
                       pool->block_size, int(row_bytes / 16));
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" int af_fp8_quantize(const void* src_f16, uint8_t* dst, size_t n, float scale,
                               af_stream_t stream) {
    if (!src_f16 || !dst || !(scale > 0.0f) || !std::isfinite(scale)) return AF_ERR_INVALID_ARG;
    if (n == 0) return AF_OK;
    hipLaunchKernelGGL(fp8_quantize_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(src_f16),
                       dst, n, scale);
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" int af_rt_fill_u32(void* dst, uint32_t value, size_t n_words, af_stream_t stream) {
    return fill_u32(dst, value, n_words, static_cast<hipStream_t>(stream));
}

extern "C" int af_rt_add_i32(int32_t* d_values, int n, int32_t delta, af_stream_t stream) {
    if (!d_values || n < 0) return AF_ERR_INVALID_ARG;
    if (n == 0) return AF_OK;
    hipLaunchKernelGGL(add_i32_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       static_cast<hipStream_t>(stream), d_values, n, delta);
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" int af_rt_fill_randn_f16(void* dst, size_t n, uint64_t seed, float stddev,
                                    af_stream_t stream) {
    if (!dst) return AF_ERR_INVALID_ARG;
    if (n == 0) return AF_OK;
    hipLaunchKernelGGL(randn_f16_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<uint16_t*>(dst), n, seed,
                       stddev);
    AF_TRY_LAUNCH();
    return AF_OK;
}

extern "C" int af_rt_fill_randn_fp8(uint8_t* dst, size_t n, uint64_t seed, float inv_scale,
                                    af_stream_t stream) {
    if (!dst) return AF_ERR_INVALID_ARG;
    if (n == 0) return AF_OK;
    hipLaunchKernelGGL(randn_fp8_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), dst, n, seed, inv_scale);
    AF_TRY_LAUNCH();
    return AF_OK;
}
