// Host-side helpers shared by the HIP backends: error mapping onto the
// reference's exception types, device matrix views, and the streamed
// native-layout weight upload (MetalRawModel::load -> device buffer,
// metal_model.cpp:698-741, metal_llm.mm:2906-2988, moe_llm.mm:824-903).
#pragma once

#include "../kernels/common.h"
#include "gguf_reader.h"
#include "profile.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace llm {

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Kernel launcher status -> the reference's exception type.
// A profiling session (if any) sees every successful launcher call.
inline void launch_check(int status, const char* what) {
    if (status == hipllm::kOk) {
        if (RunProfiler* p = active_run_profiler()) p->on_launch(what);
        return;
    }
    if (status == hipllm::kInvalidArgument) {
        throw std::invalid_argument(std::string(what) + ": invalid kernel arguments");
    }
    if (status == hipllm::kLengthError) throw std::length_error(std::string(what) + ": shape exceeds kernel limits");
    throw std::runtime_error(std::string(what) + ": kernel launch failed: " + hipGetErrorString(hipGetLastError()));
}

inline std::size_t align_up(std::size_t v, std::size_t a) { return (v + a - 1) / a * a; }

// A weight matrix resident in the device arena in its native GGUF rows. For
// expert tensors `rows` is the rows of one expert and `expert_stride` the
// bytes between consecutive experts.
struct DevMatrix {
    const std::uint8_t* ptr = nullptr;
    std::uint32_t type = 0;
    std::size_t rows = 0;
    std::size_t cols = 0;
    std::size_t row_bytes = 0;
    std::size_t expert_stride = 0;
    const void* x16 = nullptr;  // x16 tile-packed copy for decode GEMVs, when made
};

// Q4_K / Q6_K matrices whose rows hold whole 256-value super-blocks (and the
// row alignment the packer reads) can get an x16 tile-packed copy.
inline bool x16_packable(const DevMatrix& m) {
    return m.cols % 256 == 0 && ((m.type == hipllm::kQ4_K && m.row_bytes % 16 == 0) ||
                                 (m.type == hipllm::kQ6_K && m.row_bytes % 2 == 0));
}

// Plans the device weight arena (every tensor 256-byte aligned, or packed
// right after its predecessor when requested so matching matrices can be
// multiplied as one), then streams each tensor's native bytes through two
// pinned staging buffers into one allocation.
class WeightArena {
public:
    struct Item {
        TensorDescriptor t;
        std::size_t offset = 0;
    };

    // Takes the tensor from the reader (shape-checked, consumed once) and
    // reserves its bytes; returns its index.
    std::size_t place(GgufReader& reader, const std::string& name, std::size_t rows, std::size_t cols,
                      bool pack_after_previous = false) {
        Item it;
        it.t = reader.take(name, rows, cols);
        const bool packed = pack_after_previous && !items_.empty() && items_.back().t.type == it.t.type;
        cursor_ = packed ? cursor_ : align_up(cursor_, 256);
        it.offset = cursor_;
        cursor_ += it.t.byte_size;
        items_.push_back(std::move(it));
        return items_.size() - 1;
    }

    // True when item b starts right where item a ends (one matrix of rows a + b).
    bool contiguous(std::size_t a, std::size_t b) const {
        return items_[a].t.type == items_[b].t.type && items_[b].offset == items_[a].offset + items_[a].t.byte_size;
    }

    const TensorDescriptor& tensor(std::size_t i) const { return items_[i].t; }
    std::size_t payload_bytes() const {
        std::size_t total = 0;
        for (const Item& it : items_) total += it.t.byte_size;
        return total;
    }

    void upload(GgufReader& reader, hipStream_t stream) {
        // 4 KiB of tail padding: realigned dword reads of 2-byte-aligned
        // blocks may touch up to 20 bytes past a tensor's last byte.
        bytes_ = align_up(cursor_, 256) + 4096;
        hip_check(hipMalloc(reinterpret_cast<void**>(&base_), bytes_), "hipMalloc(weights)");
        hip_check(hipMemsetAsync(base_, 0, bytes_, stream), "hipMemsetAsync(weights)");
        const std::size_t stage_bytes = 64u << 20;
        void* stage[2] = {nullptr, nullptr};
        hipEvent_t done[2] = {nullptr, nullptr};
        struct Cleanup {
            void** s;
            hipEvent_t* e;
            ~Cleanup() {
                for (int i = 0; i < 2; ++i) {
                    if (e[i]) hipEventSynchronize(e[i]), hipEventDestroy(e[i]);
                    if (s[i]) hipHostFree(s[i]);
                }
            }
        } cleanup{stage, done};
        for (int i = 0; i < 2; ++i) {
            hip_check(hipHostMalloc(&stage[i], stage_bytes, hipHostMallocDefault), "hipHostMalloc(staging)");
            hip_check(hipEventCreateWithFlags(&done[i], hipEventDisableTiming), "hipEventCreate");
        }
        int slot = 0;
        bool used[2] = {false, false};
        for (const Item& it : items_) {
            std::size_t off = 0;
            while (off < it.t.byte_size) {
                const std::size_t n = std::min(stage_bytes, it.t.byte_size - off);
                if (used[slot]) hip_check(hipEventSynchronize(done[slot]), "hipEventSynchronize(staging)");
                reader.read(it.t, off, stage[slot], n);
                hip_check(hipMemcpyAsync(base_ + it.offset + off, stage[slot], n, hipMemcpyHostToDevice, stream),
                          "hipMemcpyAsync(weights)");
                hip_check(hipEventRecord(done[slot], stream), "hipEventRecord");
                used[slot] = true;
                slot ^= 1;
                off += n;
            }
        }
        hip_check(hipStreamSynchronize(stream), "weight upload");
    }

    DevMatrix matrix(std::size_t i, std::size_t experts = 0) const {
        const TensorDescriptor& t = items_[i].t;
        DevMatrix m;
        m.ptr = base_ + items_[i].offset;
        m.type = static_cast<std::uint32_t>(t.type);
        m.cols = t.cols;
        m.row_bytes = t.row_bytes;
        m.rows = experts ? t.rows / experts : t.rows;
        m.expert_stride = experts ? m.rows * t.row_bytes : 0;
        return m;
    }
    const float* vec(std::size_t i) const { return reinterpret_cast<const float*>(base_ + items_[i].offset); }

    std::uint8_t* base() const { return base_; }
    void release() {
        if (base_) hipFree(base_);
        base_ = nullptr;
    }

private:
    std::vector<Item> items_;
    std::size_t cursor_ = 0;
    std::uint8_t* base_ = nullptr;
    std::size_t bytes_ = 0;
};

}  // namespace llm
