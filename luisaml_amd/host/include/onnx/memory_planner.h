// memory_planner.h -- device-memory planning for a graph's intermediates.
//
// The reference assigns its intermediates to shader-local registers with an
// interference graph of live ranges and a size-aware greedy colouring
// (src/onnx/register_allocator/register_allocator.cpp: live ranges 589-633,
// interference 649-680, colouring 685-...).  Here the same question is asked
// of device memory: every intermediate is live from the node that writes it
// through the last node that reads it (schedule order), and two buffers may
// share bytes only when their live ranges are disjoint.  The plan places the
// buffers in one arena, largest first, each at the best-fitting gap among the
// buffers it interferes with.
#pragma once

#include <cstddef>
#include <vector>

namespace lcml::onnx {

struct BufferRequest {
    size_t bytes;
    size_t first, last;  // live over nodes [first, last] (inclusive)
};

struct MemoryPlan {
    std::vector<size_t> offsets;  // byte offset of each request in the arena
    size_t arena_bytes = 0;       // the arena's size
    size_t unshared_bytes = 0;    // the sum of the (aligned) request sizes
};

// Offsets are multiples of `alignment` (a power of two).
MemoryPlan plan_device_buffers(const std::vector<BufferRequest> &requests, size_t alignment = 256);

// true when no two requests with overlapping live ranges overlap in memory
bool plan_is_valid(const std::vector<BufferRequest> &requests, const MemoryPlan &plan);

}  // namespace lcml::onnx
