#pragma once
// AtomFlow .bin weight format and loader.
//
// Format (written by tools/quantize_weights.py:320-427, read by
// include/memory/weight_loader.h:23-130 and src/core/engine.cu:97-148 of the
// reference), little-endian, every block padded with zeros to a multiple of
// 256 bytes:
//   header (256 B): "ATOM", version, group_size, dim, hidden_dim, n_layers,
//                   n_heads, n_kv_heads, vocab_size, max_seq_len (int32 each)
//   embed_tokens    fp32 [vocab, dim]
//   per layer:      input_layernorm fp32 [dim], post_attention_layernorm fp32 [dim],
//                   then for qkv [q+2kv, dim], o_proj [dim, dim], gate [ffn, dim],
//                   up [ffn, dim], down [dim, ffn]: E4M3 codes [N, K] then fp16
//                   scales [N, K/group_size] (absmax/448 per group of group_size)
//   model.norm      fp32 [dim]
//   lm_head         fp16 [vocab, dim]
// q = dim, kv = n_kv_heads * dim / n_heads.
//
// WeightLoader keeps the reference's class (mmap, header, a cursor with
// next_block / next<T>) and adds the layout of every tensor and one streamed
// upload: the payload after the header is copied to device memory as a single
// block through pinned double buffers, so each tensor is the device view at its
// file offset (256-B aligned) and no per-tensor copy is made.
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "af_kv.h"
#include "core/view.h"

// Reference: weight_loader.h:17-19 (kept global, as callers use it unqualified).
inline size_t align_up(size_t size, size_t alignment = 256) {
    return (size + alignment - 1) & ~(alignment - 1);
}

// Reference: weight_loader.h:23-34, the Python struct.pack layout.
struct AtomHeader {
    char magic[4];
    int version;
    int group_size;
    int dim;
    int hidden_dim;
    int n_layers;
    int n_heads;
    int n_kv_heads;
    int vocab_size;
    int max_seq_len;
};
static_assert(sizeof(AtomHeader) == 40, "AtomHeader must match the packed file header");

namespace atomflow {

// Tensor kinds in file order within a layer.
enum class WeightKind : int {
    Embed = 0,
    InputNorm,
    PostNorm,
    Qkv,
    QkvScales,
    OProj,
    OProjScales,
    Gate,
    GateScales,
    Up,
    UpScales,
    Down,
    DownScales,
    FinalNorm,
    LmHead,
};

struct TensorSpec {
    WeightKind kind;
    int layer;       // -1 for model-level tensors
    DataType dtype;
    int64_t rows;    // dims: [rows, cols] (cols = 1 for vectors)
    int64_t cols;
    size_t offset;   // from the start of the file
    size_t bytes;    // unpadded
};

// Every tensor of a file with this header, in file order. Throws
// std::invalid_argument for a header the format cannot describe.
std::vector<TensorSpec> atom_layout(const AtomHeader& h);
// End of the last tensor's padded block: the least valid file size.
size_t atom_file_bytes(const AtomHeader& h);

}  // namespace atomflow

class WeightLoader {
public:
    AtomHeader header;

    // Maps the file read-only and checks the magic (weight_loader.h:52-95), the
    // header fields and that the file holds every tensor of the layout; throws
    // std::runtime_error otherwise.
    explicit WeightLoader(const std::string& filepath);
    ~WeightLoader();
    WeightLoader(const WeightLoader&) = delete;
    WeightLoader& operator=(const WeightLoader&) = delete;

    // Reference cursor API (weight_loader.h:105-129): the pointer at the cursor,
    // then the cursor moves by align_up(size_in_bytes); throws past the end.
    const void* next_block(size_t size_in_bytes);
    template <typename T>
    const T* next(size_t num_elements) {
        return static_cast<const T*>(next_block(num_elements * sizeof(T)));
    }
    size_t current_offset() const { return cursor_; }
    size_t file_size() const { return file_size_; }

    // Additions.
    const uint8_t* data() const { return base_; }
    const std::vector<atomflow::TensorSpec>& layout() const { return layout_; }
    const atomflow::TensorSpec& tensor(atomflow::WeightKind kind, int layer = -1) const;
    size_t payload_bytes() const { return file_size_ - 256; }
    // Copies the payload (file bytes [256, file_size)) to dst (>= payload_bytes())
    // through two pinned staging buffers of chunk_bytes on `stream` (a
    // hipStream_t), overlapping the host-side reads with the transfers.
    // Synchronous on return. Returns a hipError_t value (0 = success).
    int upload(void* dst, af_stream_t stream, size_t chunk_bytes = size_t(64) << 20) const;
    // The device View of a tensor inside an uploaded payload at `base`.
    View device_view(const void* base, atomflow::WeightKind kind, int layer = -1) const;

private:
    int fd_ = -1;
    size_t file_size_ = 0;
    uint8_t* base_ = nullptr;
    size_t cursor_ = 256;
    std::vector<atomflow::TensorSpec> layout_;
};
