// Row RMSNorm as a block-level device function, shared by the standalone
// kernel and kernels that finish a row and normalise it in the same block.
//
// RMSNorm follows CPULLM's Vector::rmsnorm (cpu_llm.cpp:143-166): double sum
// of squares, y = x * (inv_rms * gamma), inv_rms = 1 / sqrt(mean + eps) in
// FP32.
#pragma once

#include "common.h"

namespace hipllm {

// Normalises one row with the calling block (blockDim.x <= 1024), writing y
// and, when yq != nullptr (cols % 16 == 0), its XGroup form. cols % 4 == 0
// rows use 128-bit accesses (x, gamma and y then 16-byte aligned).
// Whole 16-groups held in registers: every thread loads its (up to) two
// groups of x and gamma at once, so the row costs one round trip to memory,
// the block reduction and the writes. yr (nullable) receives y, yq
// (nullable, global or LDS) its XGroup form. Callers with the same block size
// get identical bits (the GEMVs that normalise their input in a prologue run
// this with 256 threads, as the standalone kernel does).
__device__ inline void rmsnorm_row_groups(const float* __restrict__ xr, const float* __restrict__ gamma,
                                          float* __restrict__ yr, XGroup* yq, uint32_t cols, float eps) {
    constexpr int NG = 2;
    const uint32_t groups = cols / 16;
    float4 xv[NG][4], gv[NG][4];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        const uint32_t g = threadIdx.x + j * blockDim.x;
        if (g < groups) {
            const float4* x4 = reinterpret_cast<const float4*>(xr + 16 * g);
            const float4* g4 = reinterpret_cast<const float4*>(gamma + 16 * g);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xv[j][i] = x4[i];
                gv[j][i] = g4[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) xv[j][i] = gv[j][i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = xv[j][i];
            ss += static_cast<double>(v.x) * v.x + static_cast<double>(v.y) * v.y +
                  static_cast<double>(v.z) * v.z + static_cast<double>(v.w) * v.w;
        }
    }
    ss = wave_sum_d(ss);
    __shared__ double part[16];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    double t = 0.0;
    for (uint32_t w = 0; w < (blockDim.x + 63) / 64; ++w) t += part[w];
    const float ms = static_cast<float>(t / static_cast<double>(cols));
    const float inv = 1.0f / sqrtf(ms + eps);
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        const uint32_t g = threadIdx.x + j * blockDim.x;
        if (g >= groups) continue;
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 a = xv[j][i], b = gv[j][i];
            const float4 o = make_float4(a.x * (inv * b.x), a.y * (inv * b.y), a.z * (inv * b.z), a.w * (inv * b.w));
            if (yr) reinterpret_cast<float4*>(yr + 16 * g)[i] = o;
            v[4 * i] = o.x;
            v[4 * i + 1] = o.y;
            v[4 * i + 2] = o.z;
            v[4 * i + 3] = o.w;
        }
        if (yq) xgroup_encode(v, yq + g);
    }
}

// rmsnorm_row_groups' outputs with few live registers: x is read twice (sum
// of squares, then scale and encode), each group transiently, in the same
// order, so the bits are the same. yr (values) and yq (XGroup form) are
// nullable, global or LDS; cols % 16 == 0. For kernels that normalise their
// input in a prologue while other loads are in flight.
__device__ inline void rmsnorm_row_lean(const float* __restrict__ xr, const float* __restrict__ gamma, float* yr,
                                        XGroup* yq, uint32_t cols, float eps) {
    const uint32_t groups = cols / 16;
    double ss = 0.0;
    for (uint32_t g = threadIdx.x; g < groups; g += blockDim.x) {
        const float4* x4 = reinterpret_cast<const float4*>(xr + 16 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = x4[i];
            ss += static_cast<double>(v.x) * v.x + static_cast<double>(v.y) * v.y +
                  static_cast<double>(v.z) * v.z + static_cast<double>(v.w) * v.w;
        }
    }
    ss = wave_sum_d(ss);
    __shared__ double part[16];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    double t = 0.0;
    for (uint32_t w = 0; w < (blockDim.x + 63) / 64; ++w) t += part[w];
    const float ms = static_cast<float>(t / static_cast<double>(cols));
    const float inv = 1.0f / sqrtf(ms + eps);
    for (uint32_t g = threadIdx.x; g < groups; g += blockDim.x) {
        const float4* x4 = reinterpret_cast<const float4*>(xr + 16 * g);
        const float4* g4 = reinterpret_cast<const float4*>(gamma + 16 * g);
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 a = x4[i], b = g4[i];
            v[4 * i] = a.x * (inv * b.x);
            v[4 * i + 1] = a.y * (inv * b.y);
            v[4 * i + 2] = a.z * (inv * b.z);
            v[4 * i + 3] = a.w * (inv * b.w);
        }
        if (yr) {
            float4* y4 = reinterpret_cast<float4*>(yr + 16 * g);
#pragma unroll
            for (int i = 0; i < 4; ++i) y4[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
        }
        if (yq) xgroup_encode(v, yq + g);
    }
}

__device__ inline void rmsnorm_row(const float* __restrict__ xr, const float* __restrict__ gamma,
                                   float* __restrict__ yr, XGroup* __restrict__ yq, uint32_t cols, float eps) {
    const uint32_t groups = cols / 16;
    if (cols % 16 == 0 && groups <= 2 * blockDim.x) {
        rmsnorm_row_groups(xr, gamma, yr, yq, cols, eps);
        return;
    }
    const bool vec = (cols % 4 == 0);
    double ss = 0.0;
    if (vec) {
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        for (uint32_t i = threadIdx.x; i < cols / 4; i += blockDim.x) {
            const float4 v = x4[i];
            ss += static_cast<double>(v.x) * v.x + static_cast<double>(v.y) * v.y +
                  static_cast<double>(v.z) * v.z + static_cast<double>(v.w) * v.w;
        }
    } else {
        for (uint32_t i = threadIdx.x; i < cols; i += blockDim.x) {
            const double v = xr[i];
            ss += v * v;
        }
    }
    ss = wave_sum_d(ss);
    __shared__ double part[16];
    __shared__ float inv_s;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (uint32_t w = 0; w < (blockDim.x + 63) / 64; ++w) t += part[w];
        const float ms = static_cast<float>(t / static_cast<double>(cols));
        inv_s = 1.0f / sqrtf(ms + eps);
    }
    __syncthreads();
    const float inv = inv_s;
    if (vec) {
        for (uint32_t g = threadIdx.x; g < groups; g += blockDim.x) {
            const float4* x4 = reinterpret_cast<const float4*>(xr + 16 * g);
            const float4* g4 = reinterpret_cast<const float4*>(gamma + 16 * g);
            float4* y4 = reinterpret_cast<float4*>(yr + 16 * g);
            float v[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 a = x4[i], b = g4[i];
                const float4 o = make_float4(a.x * (inv * b.x), a.y * (inv * b.y), a.z * (inv * b.z), a.w * (inv * b.w));
                y4[i] = o;
                v[4 * i] = o.x;
                v[4 * i + 1] = o.y;
                v[4 * i + 2] = o.z;
                v[4 * i + 3] = o.w;
            }
            if (yq) xgroup_encode(v, yq + g);
        }
        for (uint32_t c = groups * 16 + threadIdx.x; c < cols; c += blockDim.x) yr[c] = xr[c] * (inv * gamma[c]);
    } else {
        for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) yr[c] = xr[c] * (inv * gamma[c]);
    }
}

}  // namespace hipllm
