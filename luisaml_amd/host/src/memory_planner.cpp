// memory_planner.cpp -- see include/onnx/memory_planner.h.
#include "onnx/memory_planner.h"

#include <algorithm>
#include <numeric>

namespace lcml::onnx {

namespace {
size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
bool lives_overlap(const BufferRequest &a, const BufferRequest &b) { return a.first <= b.last && b.first <= a.last; }
}  // namespace

MemoryPlan plan_device_buffers(const std::vector<BufferRequest> &requests, size_t alignment) {
    const size_t n = requests.size();
    MemoryPlan plan;
    plan.offsets.assign(n, 0);
    std::vector<size_t> bytes(n);
    for (size_t i = 0; i < n; ++i) {
        bytes[i] = align_up(requests[i].bytes ? requests[i].bytes : 1, alignment);
        plan.unshared_bytes += bytes[i];
    }
    // largest first; equal sizes in schedule order
    std::vector<size_t> order(n);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
        if (bytes[a] != bytes[b]) return bytes[a] > bytes[b];
        return requests[a].first < requests[b].first;
    });
    std::vector<size_t> placed;
    struct Span {
        size_t lo, hi;
    };
    std::vector<Span> busy;
    for (size_t r : order) {
        // memory taken, during r's live range, by the buffers already placed
        busy.clear();
        for (size_t p : placed)
            if (lives_overlap(requests[r], requests[p])) busy.push_back({plan.offsets[p], plan.offsets[p] + bytes[p]});
        std::sort(busy.begin(), busy.end(), [](const Span &a, const Span &b) { return a.lo < b.lo; });
        // best fit: the smallest free gap that holds r; else past the last
        size_t best = SIZE_MAX, best_gap = SIZE_MAX, cursor = 0;
        for (const Span &s : busy) {
            if (s.lo > cursor) {
                const size_t gap = s.lo - cursor;
                if (gap >= bytes[r] && gap < best_gap) {
                    best = cursor;
                    best_gap = gap;
                }
            }
            cursor = std::max(cursor, s.hi);
        }
        plan.offsets[r] = best != SIZE_MAX ? best : cursor;
        plan.arena_bytes = std::max(plan.arena_bytes, plan.offsets[r] + bytes[r]);
        placed.push_back(r);
    }
    return plan;
}

bool plan_is_valid(const std::vector<BufferRequest> &requests, const MemoryPlan &plan) {
    for (size_t i = 0; i < requests.size(); ++i) {
        if (plan.offsets[i] + requests[i].bytes > plan.arena_bytes) return false;
        for (size_t j = i + 1; j < requests.size(); ++j) {
            if (!lives_overlap(requests[i], requests[j])) continue;
            const size_t ai = plan.offsets[i], bi = ai + requests[i].bytes;
            const size_t aj = plan.offsets[j], bj = aj + requests[j].bytes;
            if (ai < bj && aj < bi && requests[i].bytes && requests[j].bytes) return false;
        }
    }
    return true;
}

}  // namespace lcml::onnx
