// weight_loader.cpp — AtomFlow .bin layout, mmap loader and streamed device
// upload (include/memory/weight_loader.h), and its C ABI (af_weights_*).
#include "memory/weight_loader.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <thread>

#include <hip/hip_runtime.h>

#include "af_kv.h"

namespace atomflow {

std::vector<TensorSpec> atom_layout(const AtomHeader& h) {
    if (std::memcmp(h.magic, "ATOM", 4) != 0) throw std::invalid_argument("not an AtomFlow header");
    if (h.group_size <= 0 || h.dim <= 0 || h.hidden_dim <= 0 || h.n_layers <= 0 ||
        h.n_heads <= 0 || h.n_kv_heads <= 0 || h.vocab_size <= 0 || h.dim % h.n_heads ||
        h.n_heads % h.n_kv_heads || h.dim % h.group_size || h.hidden_dim % h.group_size)
        throw std::invalid_argument("AtomFlow header: inconsistent model dimensions");
    const int64_t D = h.dim, F = h.hidden_dim, V = h.vocab_size, GS = h.group_size;
    const int64_t kv = int64_t(h.n_kv_heads) * (D / h.n_heads);
    const int64_t qkv = D + 2 * kv;
    std::vector<TensorSpec> out;
    size_t off = 256;
    auto put = [&](WeightKind k, int layer, DataType t, int64_t r, int64_t c) {
        const size_t bytes = size_t(r) * size_t(c) * dtype_size(t);
        out.push_back({k, layer, t, r, c, off, bytes});
        off += align_up(bytes);
    };
    auto fp8 = [&](WeightKind w, WeightKind s, int layer, int64_t n, int64_t k) {
        put(w, layer, DataType::FP8_E4M3, n, k);
        put(s, layer, DataType::FP16, n, k / GS);
    };
    put(WeightKind::Embed, -1, DataType::FP32, V, D);
    for (int l = 0; l < h.n_layers; ++l) {
        put(WeightKind::InputNorm, l, DataType::FP32, D, 1);
        put(WeightKind::PostNorm, l, DataType::FP32, D, 1);
        fp8(WeightKind::Qkv, WeightKind::QkvScales, l, qkv, D);
        fp8(WeightKind::OProj, WeightKind::OProjScales, l, D, D);
        fp8(WeightKind::Gate, WeightKind::GateScales, l, F, D);
        fp8(WeightKind::Up, WeightKind::UpScales, l, F, D);
        fp8(WeightKind::Down, WeightKind::DownScales, l, D, F);
    }
    put(WeightKind::FinalNorm, -1, DataType::FP32, D, 1);
    put(WeightKind::LmHead, -1, DataType::FP16, V, D);
    return out;
}

size_t atom_file_bytes(const AtomHeader& h) {
    const auto l = atom_layout(h);
    return l.back().offset + align_up(l.back().bytes);
}

}  // namespace atomflow

using atomflow::TensorSpec;
using atomflow::WeightKind;

WeightLoader::WeightLoader(const std::string& filepath) {
    fd_ = ::open(filepath.c_str(), O_RDONLY);
    if (fd_ == -1) throw std::runtime_error("Failed to open weights file: " + filepath);
    struct stat sb;
    if (fstat(fd_, &sb) == -1) {
        ::close(fd_);
        throw std::runtime_error("Failed to stat weights file.");
    }
    file_size_ = size_t(sb.st_size);
    if (file_size_ < 256) {
        ::close(fd_);
        throw std::runtime_error("Weight file shorter than its 256-byte header.");
    }
    void* m = mmap(nullptr, file_size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (m == MAP_FAILED) {
        ::close(fd_);
        throw std::runtime_error("Failed to mmap weights file.");
    }
    base_ = static_cast<uint8_t*>(m);
    madvise(m, file_size_, MADV_SEQUENTIAL);
    std::memcpy(&header, base_, sizeof(header));
    try {
        if (std::memcmp(header.magic, "ATOM", 4) != 0)
            throw std::runtime_error("Invalid magic number — not an AtomFlow .bin file.");
        layout_ = atomflow::atom_layout(header);
    } catch (const std::invalid_argument& e) {
        munmap(base_, file_size_);
        ::close(fd_);
        throw std::runtime_error(e.what());
    } catch (...) {
        munmap(base_, file_size_);
        ::close(fd_);
        throw;
    }
    const TensorSpec& last = layout_.back();
    if (last.offset + last.bytes > file_size_) {
        munmap(base_, file_size_);
        ::close(fd_);
        throw std::runtime_error("Weight file truncated: the layout needs " +
                                 std::to_string(last.offset + last.bytes) + " bytes, file has " +
                                 std::to_string(file_size_));
    }
}

WeightLoader::~WeightLoader() {
    if (base_) munmap(base_, file_size_);
    if (fd_ != -1) ::close(fd_);
}

const void* WeightLoader::next_block(size_t size_in_bytes) {
    const size_t at = cursor_;
    if (at + align_up(size_in_bytes) > file_size_)
        throw std::runtime_error("Weight file EOF reached unexpectedly — alignment mismatch?");
    cursor_ += align_up(size_in_bytes);
    return base_ + at;
}

const TensorSpec& WeightLoader::tensor(WeightKind kind, int layer) const {
    for (const TensorSpec& t : layout_)
        if (t.kind == kind && t.layer == layer) return t;
    throw std::out_of_range("WeightLoader: no such tensor");
}

View WeightLoader::device_view(const void* base, WeightKind kind, int layer) const {
    const TensorSpec& t = tensor(kind, layer);
    void* p = const_cast<char*>(static_cast<const char*>(base)) + (t.offset - 256);
    if (t.cols == 1) return create_contiguous_view(p, t.dtype, {t.rows});
    return create_contiguous_view(p, t.dtype, {t.rows, t.cols});
}

// Host-side copy of one chunk into pinned memory with a few threads (the page
// cache feeds one thread at well under the transfer rate).
static void parallel_copy(uint8_t* dst, const uint8_t* src, size_t n) {
    const int kThreads = 4;
    const size_t part = align_up((n + kThreads - 1) / kThreads, 4096);
    std::thread th[kThreads];
    int used = 0;
    for (int i = 0; i < kThreads; ++i) {
        const size_t b = size_t(i) * part;
        if (b >= n) break;
        const size_t e = std::min(n, b + part);
        th[used++] = std::thread([=] { std::memcpy(dst + b, src + b, e - b); });
    }
    for (int i = 0; i < used; ++i) th[i].join();
}

int WeightLoader::upload(void* dst, af_stream_t stream_handle, size_t chunk_bytes) const {
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    if (!dst || chunk_bytes == 0) return int(hipErrorInvalidValue);
    const size_t total = payload_bytes();
    uint8_t* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        e = hipHostMalloc(reinterpret_cast<void**>(&stage[i]), chunk_bytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
    }
    bool used[2] = {false, false};
    for (size_t off = 0, k = 0; e == hipSuccess && off < total; off += chunk_bytes, ++k) {
        const int b = int(k & 1);
        const size_t n = std::min(chunk_bytes, total - off);
        if (used[b]) e = hipEventSynchronize(done[b]);  // the buffer's previous copy is done
        if (e != hipSuccess) break;
        parallel_copy(stage[b], base_ + 256 + off, n);
        e = hipMemcpyAsync(static_cast<uint8_t*>(dst) + off, stage[b], n, hipMemcpyHostToDevice,
                           stream);
        if (e == hipSuccess) e = hipEventRecord(done[b], stream);
        used[b] = true;
    }
    const hipError_t s = hipStreamSynchronize(stream);
    if (e == hipSuccess) e = s;
    for (int i = 0; i < 2; ++i) {
        if (done[i]) (void)hipEventDestroy(done[i]);
        if (stage[i]) (void)hipHostFree(stage[i]);
    }
    return int(e);
}

// ============================================================================
// C ABI
// ============================================================================
struct af_weights {
    WeightLoader loader;
    explicit af_weights(const char* path) : loader(path) {}
};

extern "C" int af_weights_open(const char* path, af_weights** out) {
    if (!path || !out) return AF_ERR_INVALID_ARG;
    *out = nullptr;
    try {
        *out = new af_weights(path);
    } catch (const std::bad_alloc&) {
        return AF_ERR_INVALID_ARG;
    } catch (const std::exception&) {
        return AF_ERR_BAD_FILE;
    }
    return AF_OK;
}

extern "C" size_t af_weights_layout_bytes(const int32_t* fields) {
    if (!fields) return 0;
    AtomHeader h;
    std::memcpy(h.magic, "ATOM", 4);
    h.version = fields[0];
    h.group_size = fields[1];
    h.dim = fields[2];
    h.hidden_dim = fields[3];
    h.n_layers = fields[4];
    h.n_heads = fields[5];
    h.n_kv_heads = fields[6];
    h.vocab_size = fields[7];
    h.max_seq_len = fields[8];
    try {
        return atomflow::atom_file_bytes(h);
    } catch (const std::exception&) {
        return 0;
    }
}

extern "C" int af_weights_close(af_weights* w) {
    delete w;
    return AF_OK;
}

extern "C" int af_weights_header(const af_weights* w, int32_t* fields) {
    if (!w || !fields) return AF_ERR_INVALID_ARG;
    const AtomHeader& h = w->loader.header;
    const int32_t f[9] = {h.version, h.group_size, h.dim, h.hidden_dim, h.n_layers,
                          h.n_heads, h.n_kv_heads, h.vocab_size, h.max_seq_len};
    std::memcpy(fields, f, sizeof(f));
    return AF_OK;
}

extern "C" size_t af_weights_payload_bytes(const af_weights* w) {
    return w ? w->loader.payload_bytes() : 0;
}

extern "C" int af_weights_tensor(const af_weights* w, int kind, int layer, int64_t* offset,
                                 int64_t* bytes, int64_t* dims) {
    if (!w || kind < 0 || kind > int(WeightKind::LmHead)) return AF_ERR_INVALID_ARG;
    try {
        const TensorSpec& t = w->loader.tensor(WeightKind(kind), layer);
        if (offset) *offset = int64_t(t.offset - 256);
        if (bytes) *bytes = int64_t(t.bytes);
        if (dims) {
            dims[0] = t.rows;
            dims[1] = t.cols;
        }
    } catch (const std::exception&) {
        return AF_ERR_OUT_OF_RANGE;
    }
    return AF_OK;
}

extern "C" int af_weights_upload(const af_weights* w, void* d_dst, size_t dst_bytes,
                                 af_stream_t stream) {
    if (!w || !d_dst) return AF_ERR_INVALID_ARG;
    if (dst_bytes < w->loader.payload_bytes()) return AF_ERR_WORKSPACE;
    return w->loader.upload(d_dst, stream);
}
