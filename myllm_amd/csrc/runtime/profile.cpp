// Profiling in the reference's CSV formats (see profile.h).
#include "profile.h"

#include "../kernels/common.h"

#include <algorithm>
#include <cmath>
#include <filesystem>
#include <iomanip>
#include <limits>
#include <stdexcept>
#include <tuple>

namespace hipllm {

LaunchNotes& launch_notes() {
    thread_local LaunchNotes notes;
    return notes;
}

}  // namespace hipllm

namespace llm {
namespace {

std::uint64_t sat_add(std::uint64_t a, std::uint64_t b) {
    return b > std::numeric_limits<std::uint64_t>::max() - a ? std::numeric_limits<std::uint64_t>::max() : a + b;
}

std::uint64_t sat_mul(std::uint64_t a, std::uint64_t b) {
    return a != 0 && b > std::numeric_limits<std::uint64_t>::max() / a ? std::numeric_limits<std::uint64_t>::max()
                                                                        : a * b;
}

// Quoted only when it holds a separator, as the operator table does
// (profiler.cpp:757-781); the sidecars quote every text field
// (profiler.cpp:48-60).
std::string csv_text(const std::string& v, bool always) {
    const bool quote = always || v.find_first_of(",\"\n\r") != std::string::npos;
    if (!quote) return v;
    std::string out = "\"";
    for (char c : v) {
        if (c == '"') out.push_back('"');
        out.push_back(c);
    }
    out.push_back('"');
    return out;
}

std::string sidecar_path(const std::string& primary, const char* suffix) {
    namespace fs = std::filesystem;
    const fs::path p(primary);
    std::string stem = p.stem().string();
    if (stem.empty()) stem = "llm_profile";
    return (p.parent_path() / (stem + suffix + ".csv")).string();
}

double percentile(std::vector<double> v, double f) {
    if (v.empty()) return 0.0;
    std::sort(v.begin(), v.end());
    const double pos = f * static_cast<double>(v.size() - 1);
    const std::size_t lo = static_cast<std::size_t>(pos), hi = std::min(v.size() - 1, lo + 1);
    const double w = pos - static_cast<double>(lo);
    return v[lo] * (1.0 - w) + v[hi] * w;
}

double ms_between(std::chrono::steady_clock::time_point a, std::chrono::steady_clock::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
}

}  // namespace

OpTraffic& OpTraffic::operator+=(const OpTraffic& o) {
    flops = sat_add(flops, o.flops);
    read_bytes = sat_add(read_bytes, o.read_bytes);
    write_bytes = sat_add(write_bytes, o.write_bytes);
    temporary_bytes = sat_add(temporary_bytes, o.temporary_bytes);
    allocations = sat_add(allocations, o.allocations);
    return *this;
}

OpTraffic traffic_matmul(std::size_t m, std::size_t n, std::size_t k, bool bias) {
    OpTraffic t;
    t.flops = sat_mul(sat_mul(sat_mul(m, n), k), 2);
    t.read_bytes = sat_add(sat_mul(sat_mul(m, k), 4), sat_mul(sat_mul(k, n), 4));
    t.write_bytes = sat_mul(sat_mul(m, n), 4);
    t.temporary_bytes = t.write_bytes;
    t.allocations = sat_add(m, 1);
    if (bias) {
        t.flops = sat_add(t.flops, sat_mul(m, n));
        t.read_bytes = sat_add(t.read_bytes, sat_mul(n, 4));
    }
    return t;
}

OpTraffic traffic_gemv(std::size_t input, std::size_t output) {
    OpTraffic t;
    t.flops = sat_mul(sat_mul(input, output), 2);
    t.read_bytes = sat_add(sat_mul(sat_mul(input, output), 4), sat_mul(input, 4));
    t.write_bytes = sat_mul(output, 4);
    t.temporary_bytes = t.write_bytes;
    t.allocations = 1;
    return t;
}

OpTraffic traffic_elementwise(std::size_t elements, std::uint64_t flops_per_element, std::uint64_t reads,
                              std::uint64_t writes, std::uint64_t temporary_bytes, std::uint64_t allocations) {
    OpTraffic t;
    t.flops = sat_mul(elements, flops_per_element);
    t.read_bytes = sat_mul(sat_mul(elements, reads), 4);
    t.write_bytes = sat_mul(sat_mul(elements, writes), 4);
    t.temporary_bytes = temporary_bytes;
    t.allocations = allocations;
    return t;
}

OpTraffic traffic_copy(std::uint64_t bytes, std::uint64_t allocations) {
    OpTraffic t;
    t.read_bytes = bytes;
    t.write_bytes = bytes;
    t.temporary_bytes = bytes;
    t.allocations = allocations;
    return t;
}

GraphKernels graph_kernels(hipGraph_t graph) {
    GraphKernels g;
    std::size_t count = 0;
    if (!graph || hipGraphGetNodes(graph, nullptr, &count) != hipSuccess || count == 0) return g;
    std::vector<hipGraphNode_t> nodes(count);
    if (hipGraphGetNodes(graph, nodes.data(), &count) != hipSuccess) return g;
    for (hipGraphNode_t node : nodes) {
        hipGraphNodeType type;
        if (hipGraphNodeGetType(node, &type) != hipSuccess || type != hipGraphNodeTypeKernel) continue;
        hipKernelNodeParams p{};
        if (hipGraphKernelNodeGetParams(node, &p) != hipSuccess) continue;
        const std::uint64_t blocks = static_cast<std::uint64_t>(p.gridDim.x) * p.gridDim.y * p.gridDim.z;
        const std::uint64_t per = static_cast<std::uint64_t>(p.blockDim.x) * p.blockDim.y * p.blockDim.z;
        ++g.kernels;
        g.blocks += blocks;
        g.threads += blocks * per;
        if (blocks == 1) ++g.single_block;
    }
    return g;
}

RunProfiler*& active_run_profiler() {
    thread_local RunProfiler* p = nullptr;
    return p;
}

RunProfiler::RunProfiler(const std::string& csv_path, bool detailed, hipStream_t stream)
    : stream_(stream), detailed_(detailed) {
    if (csv_path.empty()) throw std::invalid_argument("Profile CSV path cannot be empty");
    primary_.open(csv_path, std::ios::out | std::ios::trunc);
    commands_.open(sidecar_path(csv_path, "_metal_commands"), std::ios::out | std::ios::trunc);
    kernels_.open(sidecar_path(csv_path, "_metal_kernels"), std::ios::out | std::ios::trunc);
    ops_.open(sidecar_path(csv_path, "_metal_ops"), std::ios::out | std::ios::trunc);
    if (!primary_ || !commands_ || !kernels_ || !ops_) {
        throw std::runtime_error("Cannot open profile CSV: " + csv_path);
    }
    primary_ << "record_type,forward_index,sequence_tokens,layer_index,stage,calls,time_ms,flops,read_bytes,"
                "write_bytes,temporary_bytes,logical_bytes,estimated_bytes_with_temporaries,allocations,gflops,"
                "logical_gbps,estimated_gbps,arithmetic_intensity,arithmetic_intensity_with_temporaries\n";
    commands_ << "command_index,phase,sequence_tokens,kernel_count,threadgroups,dispatched_threads,"
                 "single_threadgroup_kernels,counter_requested,counter_active,counter_status,sample_count,"
                 "timestamp_ns_per_tick,cpu_command_create_ms,cpu_encode_ms,cpu_encoder_sum_ms,"
                 "cpu_encode_unattributed_ms,cpu_commit_ms,cpu_wait_ms,cpu_counter_resolve_ms,cpu_total_ms,"
                 "commit_to_scheduled_callback_ms,commit_to_completed_callback_ms,"
                 "completed_callback_to_wait_return_ms,commit_to_gpu_start_ms,gpu_start_to_kernel_start_ms,"
                 "kernel_window_ms,kernel_end_to_gpu_end_ms,gpu_duration_ms,gpu_end_to_wait_return_ms,"
                 "sampled_kernel_ms,sampled_gap_ms,sampled_span_ms,sampled_unattributed_ms,kernel_p50_us,"
                 "kernel_p90_us,kernel_p99_us,kernel_max_us,kernel_max_operation\n";
    kernels_ << "command_index,phase,sequence_tokens,order,layer_index,head_index,operation,pipeline,value_type,"
                "m,n,k,dispatch_type,grid_x,grid_y,grid_z,threads_x,threads_y,threads_z,threadgroups,"
                "dispatched_threads,cpu_encode_us,start_timestamp,end_timestamp,gpu_duration_us,"
                "gap_from_previous_us,flops,read_bytes,write_bytes,weight_bytes,shader_read_bytes,gflops,"
                "minimum_gbps,weight_gbps,shader_requested_gbps\n";
    ops_ << "command_index,phase,sequence_tokens,operation,pipeline,value_type,calls,gpu_time_ms,gpu_percent,"
            "average_us,min_us,max_us,gap_before_ms,cpu_encode_ms,flops,read_bytes,write_bytes,weight_bytes,"
            "shader_read_bytes,gflops,minimum_gbps,weight_gbps,shader_requested_gbps\n";
    events_.resize(2, nullptr);
    for (hipEvent_t& e : events_) {
        if (hipEventCreate(&e) != hipSuccess) throw std::runtime_error("hipEventCreate(profile)");
    }
}

RunProfiler::~RunProfiler() {
    if (active_run_profiler() == this) active_run_profiler() = nullptr;
    for (const auto& [stage, total] : global_) write_primary_row("global", "", "", stage, total);
    primary_.flush();
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (hipEvent_t e : events_) {
        if (e) (void)hipEventDestroy(e);
    }
}

void RunProfiler::begin(const char* phase, std::size_t sequence_tokens, const char* stage) {
    phase_ = phase;
    stage_ = stage;
    tokens_ = sequence_tokens;
    launches_.clear();
    used_events_ = 1;
    hipllm::launch_notes().count = 0;
    host_begin_ = std::chrono::steady_clock::now();
    launch_end_ = host_begin_;
    if (hipEventRecord(events_[0], stream_) != hipSuccess) throw std::runtime_error("hipEventRecord(profile)");
    active_ = true;
    active_run_profiler() = this;
}

void RunProfiler::on_launch(const char* operation) {
    if (!active_) return;
    hipllm::LaunchNotes& notes = hipllm::launch_notes();
    Launch l;
    l.operation = operation;
    for (int i = 0; i < notes.count; ++i) {
        const hipllm::LaunchNote& n = notes.note[i];
        std::string name = n.kernel;
        if (name.size() > 2 && name.front() == '(' && name.back() == ')') name = name.substr(1, name.size() - 2);
        l.kernels += (i ? "+" : "") + name;
        const std::uint64_t blocks = static_cast<std::uint64_t>(n.grid[0]) * n.grid[1] * n.grid[2];
        l.blocks += blocks;
        l.threads += blocks * n.block[0] * n.block[1] * n.block[2];
        std::copy(n.grid, n.grid + 3, l.grid);  // the last kernel's launch shape
        std::copy(n.block, n.block + 3, l.block);
    }
    notes.count = 0;
    if (detailed_) {
        if (used_events_ >= events_.size()) {
            hipEvent_t e = nullptr;
            if (hipEventCreate(&e) != hipSuccess) throw std::runtime_error("hipEventCreate(profile)");
            events_.push_back(e);
        }
        l.event = static_cast<int>(used_events_);
        if (hipEventRecord(events_[used_events_++], stream_) != hipSuccess) {
            throw std::runtime_error("hipEventRecord(profile)");
        }
    }
    launches_.push_back(std::move(l));
    launch_end_ = std::chrono::steady_clock::now();
}

void RunProfiler::mark_gpu_end() {
    if (!active_ || (detailed_ && used_events_ > 1)) return;
    if (hipEventRecord(events_[1], stream_) != hipSuccess) throw std::runtime_error("hipEventRecord(profile)");
    gpu_end_marked_ = true;
}

void RunProfiler::end(const OpTraffic& traffic, const GraphKernels* graph) {
    if (!active_) return;
    active_ = false;
    if (active_run_profiler() == this) active_run_profiler() = nullptr;
    const auto host_end = std::chrono::steady_clock::now();
    // The GPU end: the last launch's event (detailed), else the event that
    // mark_gpu_end recorded after the forward's last launch.
    hipEvent_t last = events_[1];
    if (detailed_ && used_events_ > 1) {
        last = events_[used_events_ - 1];
    } else if (!gpu_end_marked_ && hipEventRecord(last, stream_) != hipSuccess) {
        throw std::runtime_error("hipEventRecord(profile)");
    }
    gpu_end_marked_ = false;
    const auto resolve_begin = std::chrono::steady_clock::now();
    if (hipEventSynchronize(last) != hipSuccess) throw std::runtime_error("hipEventSynchronize(profile)");
    float gpu_ms = 0.0f;
    (void)hipEventElapsedTime(&gpu_ms, events_[0], last);
    std::vector<double> starts, durations;  // ns from the forward's start
    std::vector<double> durs;
    if (detailed_) {
        double prev = 0.0;
        for (const Launch& l : launches_) {
            float t = 0.0f;
            (void)hipEventElapsedTime(&t, events_[0], events_[l.event]);
            const double ns = static_cast<double>(t) * 1.0e6;
            starts.push_back(prev);
            durations.push_back(std::max(0.0, ns - prev));
            prev = ns;
        }
    }
    const auto resolve_end = std::chrono::steady_clock::now();

    // Operator table (profiler.cpp:651-682).
    StageTotal total;
    total.calls = 1;
    total.elapsed_ns = static_cast<std::uint64_t>(
        std::chrono::duration_cast<std::chrono::nanoseconds>(host_end - host_begin_).count());
    total.traffic = traffic;
    write_primary_row("forward_total", std::to_string(forward_index_), std::to_string(tokens_), "forward.total", total);
    write_primary_row("forward_stage", std::to_string(forward_index_), std::to_string(tokens_), stage_, total);
    for (const std::string& name : {std::string("forward.total"), stage_}) {
        StageTotal& g = global_[name];
        ++g.calls;
        g.elapsed_ns = sat_add(g.elapsed_ns, total.elapsed_ns);
        g.traffic += traffic;
    }
    primary_.flush();

    // Command row (profiler.cpp:347-405).
    GraphKernels counts;
    if (graph && launches_.empty()) {
        counts = *graph;
    } else {
        for (const Launch& l : launches_) {
            const int parts = static_cast<int>(std::count(l.kernels.begin(), l.kernels.end(), '+')) + 1;
            counts.kernels += l.kernels.empty() ? 1 : parts;
            counts.blocks += l.blocks;
            counts.threads += l.threads;
            if (l.blocks == 1) ++counts.single_block;
        }
    }
    double sampled = 0.0, max_ns = 0.0;
    std::string max_op;
    for (std::size_t i = 0; i < durations.size(); ++i) {
        sampled += durations[i];
        if (durations[i] > max_ns) {
            max_ns = durations[i];
            max_op = launches_[i].operation;
        }
    }
    const double span = durations.empty() ? 0.0 : starts.back() + durations.back();
    const double encode_ms = ms_between(host_begin_, launch_end_);
    commands_ << forward_index_ << ',' << csv_text(phase_, true) << ',' << tokens_ << ',' << counts.kernels << ','
              << counts.blocks << ',' << counts.threads << ',' << counts.single_block << ','
              << (detailed_ ? 1 : 0) << ',' << (detailed_ && !durations.empty() ? 1 : 0) << ','
              << csv_text(detailed_ ? "hip events after every launch" : "not requested", true) << ','
              << (detailed_ ? used_events_ : 0) << ',' << std::fixed << std::setprecision(9) << 1.0 << ','
              << std::setprecision(6) << 0.0 << ',' << encode_ms << ',' << encode_ms << ',' << 0.0 << ',' << 0.0
              << ',' << ms_between(launch_end_, host_end) << ',' << ms_between(resolve_begin, resolve_end) << ','
              << ms_between(host_begin_, resolve_end) << ",,,,,," << static_cast<double>(gpu_ms) << ",,"
              << static_cast<double>(gpu_ms) << ",," << sampled / 1.0e6 << ',' << 0.0 << ',' << span / 1.0e6
              << ',' << (durations.empty() ? 0.0 : static_cast<double>(gpu_ms) - span / 1.0e6) << ','
              << percentile(durations, 0.50) / 1.0e3 << ',' << percentile(durations, 0.90) / 1.0e3 << ','
              << percentile(durations, 0.99) / 1.0e3 << ',' << max_ns / 1.0e3 << ',' << csv_text(max_op, true)
              << '\n';

    // Kernel rows and per-operation aggregates (profiler.cpp:229-339, 407-448).
    struct Agg {
        std::uint64_t calls = 0;
        double ns = 0.0, min_ns = std::numeric_limits<double>::infinity(), max_ns = 0.0;
    };
    std::map<std::tuple<std::string, std::string>, Agg> ops;
    for (std::size_t i = 0; i < durations.size(); ++i) {
        const Launch& l = launches_[i];
        kernels_ << forward_index_ << ',' << csv_text(phase_, true) << ',' << tokens_ << ',' << i << ",,,"
                 << csv_text(l.operation, true) << ',' << csv_text(l.kernels, true) << ',' << csv_text("", true)
                 << ",0,0,0," << csv_text("grid", true) << ',' << l.grid[0] << ',' << l.grid[1] << ',' << l.grid[2]
                 << ',' << l.block[0] << ',' << l.block[1] << ',' << l.block[2] << ',' << l.blocks << ','
                 << l.threads << ',' << std::fixed << std::setprecision(3) << 0.0 << ','
                 << static_cast<std::uint64_t>(starts[i]) << ',' << static_cast<std::uint64_t>(starts[i] + durations[i])
                 << ',' << durations[i] / 1.0e3 << ",,0,0,0,0,0,,,,\n";
        Agg& a = ops[{l.operation, l.kernels}];
        ++a.calls;
        a.ns += durations[i];
        a.min_ns = std::min(a.min_ns, durations[i]);
        a.max_ns = std::max(a.max_ns, durations[i]);
    }
    for (const auto& [key, a] : ops) {
        ops_ << forward_index_ << ',' << csv_text(phase_, true) << ',' << tokens_ << ','
             << csv_text(std::get<0>(key), true) << ',' << csv_text(std::get<1>(key), true) << ','
             << csv_text("", true) << ',' << a.calls << ',' << std::fixed << std::setprecision(6) << a.ns / 1.0e6
             << ',' << (sampled > 0.0 ? a.ns / sampled * 100.0 : 0.0) << ',' << a.ns / a.calls / 1.0e3 << ','
             << a.min_ns / 1.0e3 << ',' << a.max_ns / 1.0e3 << ',' << 0.0 << ',' << 0.0 << ",0,0,0,0,0,,,,\n";
    }
    commands_.flush();
    kernels_.flush();
    ops_.flush();
    ++forward_index_;
}

void RunProfiler::write_primary_row(const char* record_type, const std::string& forward, const std::string& sequence,
                                    const std::string& stage, const StageTotal& t) {
    const double seconds = static_cast<double>(t.elapsed_ns) / 1.0e9;
    const std::uint64_t logical = sat_add(t.traffic.read_bytes, t.traffic.write_bytes);
    const std::uint64_t estimated = sat_add(logical, t.traffic.temporary_bytes);
    const double flops = static_cast<double>(t.traffic.flops);
    primary_ << csv_text(record_type, false) << ',' << forward << ',' << sequence << ",," << csv_text(stage, false)
             << ',' << t.calls << ',' << std::fixed << std::setprecision(3)
             << static_cast<double>(t.elapsed_ns) / 1.0e6 << ',' << t.traffic.flops << ',' << t.traffic.read_bytes
             << ',' << t.traffic.write_bytes << ',' << t.traffic.temporary_bytes << ',' << logical << ','
             << estimated << ',' << t.traffic.allocations << ',' << (seconds > 0.0 ? flops / seconds / 1.0e9 : 0.0)
             << ',' << (seconds > 0.0 ? static_cast<double>(logical) / seconds / 1.0e9 : 0.0) << ','
             << (seconds > 0.0 ? static_cast<double>(estimated) / seconds / 1.0e9 : 0.0) << ','
             << (logical > 0 ? flops / static_cast<double>(logical) : 0.0) << ','
             << (estimated > 0 ? flops / static_cast<double>(estimated) : 0.0) << '\n';
}

}  // namespace llm
