// Value types the backends hand to their callers.
//
// llm::MemoryStats is the host application's own type: generate() stores
// backend.memory_stats() into GenerationStats::memory (chat.cpp:875,
// chat.h:20-39), so HipLLM must return exactly that struct. When the
// application's memory_stats.h (memory_stats.h:11-37) is on the include path
// it is used as is; a standalone build of this library defines the same
// layout (same fields, same order, same saturating total), so objects cross
// the library boundary unchanged either way.
#pragma once

#include <cstddef>
#include <cstdint>
#include <limits>
#include <string>

#if __has_include("memory_stats.h")
#include "memory_stats.h"
#else
namespace llm {

struct MemoryStats {
    std::uint64_t weight_bytes = 0;
    std::uint64_t kv_cache_bytes = 0;
    std::uint64_t recurrent_state_bytes = 0;
    std::uint64_t intermediate_bytes = 0;
    bool intermediate_is_estimate = false;

    // Sum of the four byte counts, saturating at the largest uint64 value.
    std::uint64_t total_bytes() const noexcept {
        const std::uint64_t mx = std::numeric_limits<std::uint64_t>::max();
        std::uint64_t t = weight_bytes;
        for (std::uint64_t v : {kv_cache_bytes, recurrent_state_bytes, intermediate_bytes}) {
            if (v > mx - t) return mx;
            t += v;
        }
        return t;
    }
};

}  // namespace llm
#endif

namespace llm {

// Expert lookups of a HipMoeLLM (the counterpart of MoeLLM's
// ExpertCacheStats, moe_llm.h:12-20). Every routed expert is resident in
// device memory, so every lookup is a hit.
struct HipExpertCacheStats {
    std::uint64_t hits = 0;
    std::uint64_t misses = 0;
    std::uint64_t requests() const noexcept { return hits + misses; }
};

// Device selection of a backend constructor: "" keeps the calling thread's
// current HIP device; "N" or "hip:N" selects visible device N. Throws
// std::invalid_argument for anything else.
int parse_device_spec(const std::string& spec);

}  // namespace llm
