// Device-side helpers shared by the HipLLM kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hipllm {

// GGML type ids (GGUF format, metal_model.h:14-29).
enum : uint32_t {
    kF32 = 0,
    kF16 = 1,
    kQ5_0 = 6,
    kQ8_0 = 8,
    kQ4_K = 12,
    kQ6_K = 14,
};

// Status codes shared with the C ABI; they mirror the reference's exception
// types (std::invalid_argument, out_of_range, length_error, runtime_error,
// overflow_error).
enum : int {
    kOk = 0,
    kInvalidArgument = 1,
    kOutOfRange = 2,
    kLengthError = 3,
    kRuntimeError = 4,
    kOverflowError = 5,
};

// Host side: the kernels a launcher just started (name, grid, block), kept
// per host thread for the runtime's profiler, which takes them after each
// launcher call (a few stores per launch; at most kLaunchNotes are kept).
struct LaunchNote {
    const char* kernel;
    uint32_t grid[3];
    uint32_t block[3];
};
constexpr int kLaunchNotes = 8;
struct LaunchNotes {
    LaunchNote note[kLaunchNotes];
    int count = 0;
};
LaunchNotes& launch_notes();

inline void note_launch(const char* kernel, dim3 grid, dim3 block) {
    LaunchNotes& n = launch_notes();
    if (n.count >= kLaunchNotes) return;
    n.note[n.count++] = LaunchNote{kernel, {grid.x, grid.y, grid.z}, {block.x, block.y, block.z}};
}

#define HIPLLM_LAUNCH(kernel, grid, block, shm, stream, ...)                      \
    do {                                                                          \
        ::hipllm::note_launch(#kernel, dim3(grid), dim3(block));                  \
        hipLaunchKernelGGL(kernel, grid, block, shm, stream, __VA_ARGS__);        \
    } while (0)

__host__ __device__ constexpr uint32_t block_elems(uint32_t type) {
    return type == kQ4_K || type == kQ6_K ? 256u : (type == kQ5_0 || type == kQ8_0) ? 32u : 1u;
}

__host__ __device__ constexpr uint32_t block_bytes(uint32_t type) {
    return type == kQ4_K ? 144u : type == kQ6_K ? 210u : type == kQ5_0 ? 22u
         : type == kQ8_0 ? 34u : type == kF16 ? 2u : 4u;
}

// Exact binary16 -> binary32, same results as the reference's half_to_float
// (model.cpp:500-522) including subnormals, infinities and a canonical quiet
// NaN. Built from integer operations so no rounding mode can interfere.
__device__ __forceinline__ float half_bits_to_float_exact(uint32_t h) {
    const uint32_t sign = (h >> 15) & 1u;
    const uint32_t exponent = (h >> 10) & 0x1fu;
    const uint32_t mantissa = h & 0x3ffu;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign << 31;
        } else {
            // value = mantissa * 2^-24; normalise the 10-bit mantissa.
            const int lead = 31 - __builtin_clz(mantissa);  // 0..9
            const uint32_t e = static_cast<uint32_t>(lead - 24 + 127);
            const uint32_t m = (mantissa << (23 - lead)) & 0x7fffffu;
            bits = (sign << 31) | (e << 23) | m;
        }
    } else if (exponent == 31) {
        bits = mantissa == 0 ? ((sign << 31) | 0x7f800000u) : 0x7fc00000u;
    } else {
        bits = (sign << 31) | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    return __uint_as_float(bits);
}

// Hardware conversion (v_cvt_f32_f16); identical to the exact form for every
// finite or infinite input, used on the GEMV hot path.
__device__ __forceinline__ float half_lo(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
}
__device__ __forceinline__ float half_hi(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

// Byte-granular little-endian loads from 2-byte-aligned addresses, built from
// naturally aligned dword loads and v_alignbyte. `p` must be 2-byte aligned and
// the dwords touched must be in bounds (device weight buffers carry padding).
__device__ __forceinline__ uint32_t load_u32_a2(const uint8_t* p) {
    const uint32_t shift = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p - shift);
    const uint32_t lo = q[0];
    const uint32_t hi = q[1];
    return __builtin_amdgcn_alignbyte(hi, lo, shift);
}

__device__ __forceinline__ uint2 load_u64_a2(const uint8_t* p) {
    const uint32_t shift = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p - shift);
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2];
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, shift),
                      __builtin_amdgcn_alignbyte(w2, w1, shift));
}

__device__ __forceinline__ uint4 load_u128_a2(const uint8_t* p) {
    const uint32_t shift = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p - shift);
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2], w3 = q[3], w4 = q[4];
    return make_uint4(__builtin_amdgcn_alignbyte(w1, w0, shift),
                      __builtin_amdgcn_alignbyte(w2, w1, shift),
                      __builtin_amdgcn_alignbyte(w3, w2, shift),
                      __builtin_amdgcn_alignbyte(w4, w3, shift));
}

__device__ __forceinline__ uint32_t load_u16_a2(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

// Unsigned byte k of a dword as float; the backend selects v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ float ubyte0(uint32_t w) { return static_cast<float>((w >> 0) & 0xffu); }
__device__ __forceinline__ float ubyte1(uint32_t w) { return static_cast<float>((w >> 8) & 0xffu); }
__device__ __forceinline__ float ubyte2(uint32_t w) { return static_cast<float>((w >> 16) & 0xffu); }
__device__ __forceinline__ float ubyte3(uint32_t w) { return static_cast<float>((w >> 24) & 0xffu); }

// ---------------------------------------------------------------- wave reductions
// Whole-wave reductions for uniform control flow, every lane receiving the
// result: DPP steps inside each row of 16 lanes (swap neighbours, swap pairs,
// mirror half-rows, mirror the row), after which every lane of a row holds
// the row's result, then the four row results read with v_readlane and
// combined in a fixed order. No LDS traffic and no address registers.
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int Ctrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), Ctrl, 0xf, 0xf, true));
}
template <int Ctrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __uint_as_float(dpp_u32<Ctrl>(__float_as_uint(v)));
}
template <int Ctrl>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
    const uint64_t lo = dpp_u32<Ctrl>(static_cast<uint32_t>(b));
    const uint64_t hi = dpp_u32<Ctrl>(static_cast<uint32_t>(b >> 32));
    return __longlong_as_double(static_cast<long long>(lo | (hi << 32)));
}
__device__ __forceinline__ float lane_f32(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ double lane_f64(double v, int lane) {
    const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
    const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b), lane));
    const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane));
    return __longlong_as_double(static_cast<long long>(lo | (hi << 32)));
}

// Sum over the four lanes of each quad (lanes 4i .. 4i + 3), equal in all four.
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_f32<kDppQuadXor1>(v);
    return v + dpp_f32<kDppQuadXor2>(v);
}

// Sum over each row of 16 lanes (lanes 16i .. 16i + 15), equal in all 16.
__device__ __forceinline__ float row16_sum(float v) {
    v = quad_sum(v);
    v += dpp_f32<kDppHalfMirror>(v);
    return v + dpp_f32<kDppMirror>(v);
}

__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
    v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
    v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f32<kDppMirror>(v));
    return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

__device__ __forceinline__ double wave_sum_d(double v) {
    v += dpp_f64<kDppQuadXor1>(v);
    v += dpp_f64<kDppQuadXor2>(v);
    v += dpp_f64<kDppHalfMirror>(v);
    v += dpp_f64<kDppMirror>(v);
    return (lane_f64(v, 0) + lane_f64(v, 16)) + (lane_f64(v, 32) + lane_f64(v, 48));
}

// ---------------------------------------------------------------- XGroup
// Activation format of the integer GEMV path. Every 16 consecutive values
// x[16g .. 16g + 15] of a GEMV input are held as 24-bit fixed point
// q = round(x / e) with |q| <= kXGroupMax, split into balanced base-256
// digits q = s2 * 65536 + s1 * 256 + s0 (each digit a signed byte, so that
// v_dot4_i32_i8 multiplies them with weight quants directly), together with
// the FP32 sum of the 16 values, the scale e = max|x| / kXGroupMax and the
// digit weights 256 e and 65536 e. The
// representation error |x - e q| is at most e, 2^-23 of the group's largest
// magnitude, i.e. the rounding error of FP32 itself at that magnitude; dot
// products of quants with the digits are exact integers.
constexpr float kXGroupMax = 8355711.0f;  // 0x7f7f7f: largest q whose digits all fit a signed byte

struct __align__(16) XGroup {
    uint32_t s0[4], s1[4], s2[4];  // digits, 4 values per dword, value i in byte i % 4 of dword i / 4
    float sum, e, e256, e65536;    // e256 = 256 e and e65536 = 65536 e (digit weights, exact)
};
static_assert(sizeof(XGroup) == 64, "XGroup is 64 bytes");

// Encodes 16 values held by one thread. Groups whose largest magnitude is
// below 2^-100 are stored as zero (their contribution is below FP32
// resolution of any realistic output); a non-finite value makes e NaN, so the
// GEMV outputs that read the group are NaN (FP32 would give inf or NaN).
__device__ __forceinline__ void xgroup_encode(const float (&v)[16], XGroup* __restrict__ g) {
    float sum = 0.0f, amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        sum += v[i];
        amax = fmaxf(amax, fabsf(v[i]));
    }
    // fmaxf drops NaN operands, so NaN shows in the sum instead.
    const bool finite = amax <= 3.4028234663852886e38f && sum == sum;
    const bool tiny = amax < 7.888609052210118e-31f;  // 2^-100
    const float e = finite ? (tiny ? 0.0f : amax / kXGroupMax) : __builtin_nanf("");
    const float inv = (finite && !tiny) ? kXGroupMax / amax : 0.0f;
    uint32_t w0[4] = {0, 0, 0, 0}, w1[4] = {0, 0, 0, 0}, w2[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float t = rintf(v[i] * inv);
        t = fminf(fmaxf(t, -kXGroupMax), kXGroupMax);
        const int q = static_cast<int>(t);
        const int d0 = static_cast<int>(static_cast<int8_t>(q & 0xff));
        const int r = (q - d0) >> 8;
        const int d1 = static_cast<int>(static_cast<int8_t>(r & 0xff));
        const int d2 = (r - d1) >> 8;
        const uint32_t sh = 8u * (i & 3);
        w0[i >> 2] |= (static_cast<uint32_t>(d0) & 0xffu) << sh;
        w1[i >> 2] |= (static_cast<uint32_t>(d1) & 0xffu) << sh;
        w2[i >> 2] |= (static_cast<uint32_t>(d2) & 0xffu) << sh;
    }
    uint4* o = reinterpret_cast<uint4*>(g);
    o[0] = make_uint4(w0[0], w0[1], w0[2], w0[3]);
    o[1] = make_uint4(w1[0], w1[1], w1[2], w1[3]);
    o[2] = make_uint4(w2[0], w2[1], w2[2], w2[3]);
    o[3] = make_uint4(__float_as_uint(sum), __float_as_uint(e), __float_as_uint(e * 256.0f),
                      __float_as_uint(e * 65536.0f));
}

// Encodes group g from 16 floats at src (global or LDS, 16-byte aligned).
__device__ __forceinline__ void xgroup_encode_from(const float* src, XGroup* __restrict__ g) {
    float v[16];
    const float4* p = reinterpret_cast<const float4*>(src);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 t = p[i];
        v[4 * i] = t.x;
        v[4 * i + 1] = t.y;
        v[4 * i + 2] = t.z;
        v[4 * i + 3] = t.w;
    }
    xgroup_encode(v, g);
}

}  // namespace hipllm
