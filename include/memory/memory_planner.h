#pragma once
// MemoryPlanner: typed 16-B aligned bump allocation over a caller-owned arena.
// Reference: include/memory/memory_planner.h:1-29 (same methods; throws
// std::runtime_error on overflow).
#include <cstddef>
#include <stdexcept>

class MemoryPlanner {
public:
    MemoryPlanner(void* arena, size_t size)
        : base_ptr_(static_cast<char*>(arena)), current_offset_(0), total_size_(size) {}

    template <typename T>
    T* allocate(size_t num_elements) {
        const size_t bytes = num_elements * sizeof(T);
        const size_t aligned_bytes = (bytes + 15) & ~size_t(15);
        if (current_offset_ + aligned_bytes > total_size_)
            throw std::runtime_error("Arena Out Of Memory!");
        T* ptr = reinterpret_cast<T*>(base_ptr_ + current_offset_);
        current_offset_ += aligned_bytes;
        return ptr;
    }
    void reset_to(size_t offset) { current_offset_ = offset; }
    size_t get_offset() const { return current_offset_; }

private:
    char* base_ptr_;
    size_t current_offset_;
    size_t total_size_;
};
