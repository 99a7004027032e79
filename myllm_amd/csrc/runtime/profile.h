// Profiling of the HIP backends in the reference's CSV formats.
//
// enable_profiling(csv, detailed) (metal_llm.h:38-40) writes:
// * csv: the per-forward operator table of the reference's Profiler
//   (profiler.cpp:619-632 header; rows forward_total / forward_stage per
//   forward, global rows when profiling stops), with the stage names the
//   reference backends use (prefill.gpu_resident / decode.gpu_resident for
//   qwen2, prefill.gpu_moe / decode.gpu_moe for qwen35moe) and the same
//   logical-traffic estimates (flops and FP32 tensor bytes by shape);
// * <stem>_metal_commands.csv, <stem>_metal_kernels.csv,
//   <stem>_metal_ops.csv: the reference's command / kernel / operation
//   sidecars (profiler.cpp:127-174), under the same names so that existing
//   analysis scripts read them. One command is one forward (prefill or
//   decode): kernel and block counts, host launch / wait time and the GPU
//   time between HIP events around it. With detailed = true every launch is
//   followed by a HIP event (decode steps then run eagerly, not as a replayed
//   graph, which perturbs timing as the reference's counter mode does): the
//   kernels file gets one row per launch, its operation, kernel(s), grid and
//   block, and its GPU time (from the previous event to its own, so a row
//   includes the launch gap before it), and the operations file aggregates
//   them.
#pragma once

#include <hip/hip_runtime.h>

#include <chrono>
#include <cstddef>
#include <cstdint>
#include <fstream>
#include <map>
#include <string>
#include <vector>

namespace llm {

// Logical traffic of an operator, estimated from tensor shapes (the
// semantics of the reference's ProfileMetrics, profiler.h:17-30).
struct OpTraffic {
    std::uint64_t flops = 0;
    std::uint64_t read_bytes = 0;
    std::uint64_t write_bytes = 0;
    std::uint64_t temporary_bytes = 0;
    std::uint64_t allocations = 0;
    OpTraffic& operator+=(const OpTraffic& o);
};

// Shape-based estimates with the reference's definitions
// (profiler.cpp:473-548): FP32 operands, 4 bytes per value.
OpTraffic traffic_matmul(std::size_t m, std::size_t n, std::size_t k, bool bias = false);
OpTraffic traffic_gemv(std::size_t input, std::size_t output);
OpTraffic traffic_elementwise(std::size_t elements, std::uint64_t flops_per_element, std::uint64_t reads,
                              std::uint64_t writes, std::uint64_t temporary_bytes = 0,
                              std::uint64_t allocations = 0);
OpTraffic traffic_copy(std::uint64_t bytes, std::uint64_t allocations = 0);

// Kernel counts of a recorded decode graph (reported for every replay).
struct GraphKernels {
    std::uint64_t kernels = 0;
    std::uint64_t blocks = 0;
    std::uint64_t threads = 0;
    std::uint64_t single_block = 0;
};
GraphKernels graph_kernels(hipGraph_t graph);

class RunProfiler {
public:
    RunProfiler(const std::string& csv_path, bool detailed, hipStream_t stream);
    ~RunProfiler();
    RunProfiler(const RunProfiler&) = delete;
    RunProfiler& operator=(const RunProfiler&) = delete;

    bool detailed() const noexcept { return detailed_; }

    // One forward: begin before its first launch (stage: the reference's
    // scope name), end after its result was read back. graph: the kernels of
    // a replayed graph (nullptr for launches made one by one).
    // mark_gpu_end right after the forward's last launch (before its
    // read-back synchronises the stream).
    void begin(const char* phase, std::size_t sequence_tokens, const char* stage);
    void mark_gpu_end();
    void end(const OpTraffic& traffic, const GraphKernels* graph = nullptr);

    // Called after every kernel launcher of the forward (launch_check).
    void on_launch(const char* operation);

private:
    struct Launch {
        std::string operation;
        std::string kernels;
        std::uint32_t grid[3] = {0, 0, 0};
        std::uint32_t block[3] = {0, 0, 0};
        std::uint64_t blocks = 0;
        std::uint64_t threads = 0;
        int event = -1;  // index into events_ (detailed mode)
    };
    struct StageTotal {
        std::uint64_t calls = 0;
        std::uint64_t elapsed_ns = 0;
        OpTraffic traffic;
    };
    void write_primary_row(const char* record_type, const std::string& forward, const std::string& sequence,
                           const std::string& stage, const StageTotal& total);

    std::ofstream primary_, commands_, kernels_, ops_;
    hipStream_t stream_;
    bool detailed_;
    std::vector<hipEvent_t> events_;  // [0] = forward start; grown on demand
    std::size_t used_events_ = 0;
    std::vector<Launch> launches_;
    std::map<std::string, StageTotal> global_;
    std::size_t forward_index_ = 0;
    bool active_ = false;
    bool gpu_end_marked_ = false;
    std::string phase_, stage_;
    std::size_t tokens_ = 0;
    std::chrono::steady_clock::time_point host_begin_, launch_end_;
};

// The profiler receiving this host thread's launches (nullptr: none).
RunProfiler*& active_run_profiler();

}  // namespace llm
