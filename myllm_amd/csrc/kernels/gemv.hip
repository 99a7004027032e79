// Decode GEMV over native GGUF block-quantized weights: y[N] = W[N,K] x[K].
//
// Replaces the reference's one-thread-per-row GEVMs (metal_llm.metal:708-781,
// dot_q*_f32 319-553; host encode_vector_product metal_llm.mm:1891-1999) with
// a wave-cooperative design for CDNA4:
//
// * An "octet" of 8 lanes owns one unit of a row (a 256-value super-block for
//   Q4_K / Q6_K / F32 / F16, two 32-value blocks for Q8_0 / Q5_0). Every lane
//   issues 128-bit loads of its slice of the unit, so a wave instruction
//   covers whole contiguous super-blocks.
// * A 256-thread block (4 waves, 32 octets) computes RB rows. Octet o works on
//   row o % RB, units o / RB, o / RB + 32 / RB, ... When RB >= 8 the eight
//   octets of one wave hold eight different rows at the same unit, so the
//   activation loads of a wave instruction are shared by eight rows.
// * Values are dequantized in registers to FP32 and accumulated in FP32. The
//   constant part of each affine block format (Q4_K's -dmin*m, Q6_K's -32,
//   Q8_0's -128 after the sign flip, Q5_0's -16) is applied once per group via
//   per-16 sums of x (xs16) that the activation's producer writes.
// * Octet partials reduce with lane shuffles, then across octets in LDS in a
//   fixed order (deterministic), and the epilogue adds bias and residual.
//
// Weight rows may be only 2-byte aligned (Q6_K / Q8_0 / Q5_0 block sizes are
// 210 / 34 / 22 bytes); such loads read the enclosing aligned dwords and
// realign with v_alignbyte. Device weight buffers carry 256 bytes of tail
// padding so those reads stay in bounds.
#include "common.h"

namespace hipllm {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

namespace {

__device__ __forceinline__ uint4 ld128_a4(const uint8_t* p) {
    const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes from a 2-byte-aligned address.
__device__ __forceinline__ uint4 ld128_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint8_t* base = reinterpret_cast<const uint8_t*>(a & ~uintptr_t(3));
    const uint32_t s = static_cast<uint32_t>(a & 3u);
    const uint4 v = ld128_a4(base);
    const uint32_t e = *reinterpret_cast<const uint32_t*>(base + 16);
    return make_uint4(__builtin_amdgcn_alignbyte(v.y, v.x, s), __builtin_amdgcn_alignbyte(v.z, v.y, s),
                      __builtin_amdgcn_alignbyte(v.w, v.z, s), __builtin_amdgcn_alignbyte(e, v.w, s));
}

__device__ __forceinline__ float dot4_u8(uint32_t q, float4 xv, float acc) {
    acc = fmaf(xv.x, ubyte0(q), acc);
    acc = fmaf(xv.y, ubyte1(q), acc);
    acc = fmaf(xv.z, ubyte2(q), acc);
    acc = fmaf(xv.w, ubyte3(q), acc);
    return acc;
}

__device__ __forceinline__ float4 ldx4(const float* p) { return *reinterpret_cast<const float4*>(p); }

template <uint32_t T>
struct Unit;

// Q4_K: 144-byte super-block {d, dmin, scales[12], qs[128]}. Lane c of the
// octet takes qs bytes [16c, 16c+16): group j = c/2, l0 = 16 (c & 1); its low
// nibbles are elements 64j+l0.. of sub-block 2j, its high nibbles elements
// 64j+32+l0.. of sub-block 2j+1 (model.cpp:616-644).
template <>
struct Unit<kQ4_K> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 144;
    __device__ static __forceinline__ float dot(const uint8_t* u, uint32_t c, const float* x,
                                                const float* xs16) {
        const uint4 h = ld128_a4(u);
        const uint4 q = ld128_a4(u + 16 + 16 * c);
        const uint32_t j = c >> 1;
        const uint32_t l0 = (c & 1) * 16;
        const float* xl = x + 64 * j + l0;
        const float* xh = xl + 32;
        const float4 a0 = ldx4(xl), a1 = ldx4(xl + 4), a2 = ldx4(xl + 8), a3 = ldx4(xl + 12);
        const float4 b0 = ldx4(xh), b1 = ldx4(xh + 4), b2 = ldx4(xh + 8), b3 = ldx4(xh + 12);
        const float sl = xs16[(64 * j + l0) >> 4];
        const float sh = xs16[(64 * j + 32 + l0) >> 4];
        // 6-bit scale/min pairs of all eight sub-blocks as packed bytes
        // (get_scale_min_k4, model.cpp:524-537), then this lane's two.
        uint32_t S, M;
        if (j < 2) {
            S = h.y & 0x3f3f3f3fu;
            M = h.z & 0x3f3f3f3fu;
        } else {
            S = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
            M = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
        }
        const uint32_t sh16 = (j & 1) * 16;
        S >>= sh16;
        M >>= sh16;
        const float d = half_lo(h.x);
        const float dmin = half_hi(h.x);
        float s0 = 0.0f, s1 = 0.0f;
        s0 = dot4_u8(q.x & 0x0f0f0f0fu, a0, s0);
        s1 = dot4_u8((q.x >> 4) & 0x0f0f0f0fu, b0, s1);
        s0 = dot4_u8(q.y & 0x0f0f0f0fu, a1, s0);
        s1 = dot4_u8((q.y >> 4) & 0x0f0f0f0fu, b1, s1);
        s0 = dot4_u8(q.z & 0x0f0f0f0fu, a2, s0);
        s1 = dot4_u8((q.z >> 4) & 0x0f0f0f0fu, b2, s1);
        s0 = dot4_u8(q.w & 0x0f0f0f0fu, a3, s0);
        s1 = dot4_u8((q.w >> 4) & 0x0f0f0f0fu, b3, s1);
        const float r0 = d * ubyte0(S) * s0 - dmin * ubyte0(M) * sl;
        const float r1 = d * ubyte1(S) * s1 - dmin * ubyte1(M) * sh;
        return r0 + r1;
    }
};

// Q6_K: 210-byte super-block {ql[128], qh[64], scales[16] int8, d}. Lane
// c = (n, m, h) takes ql bytes [64n + 32m + 16h, +16) and qh bytes
// [32n + 16h, +16): its low nibbles are elements 128n + 32m + 16h + l and its
// high nibbles elements 128n + 64 + 32m + 16h + l (model.cpp:646-683), each a
// 16-group with one int8 scale.
template <>
struct Unit<kQ6_K> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 210;
    __device__ static __forceinline__ float dot(const uint8_t* u, uint32_t c, const float* x,
                                                const float* xs16) {
        const uint32_t n = c >> 2, m = (c >> 1) & 1, hh = c & 1;
        const uint4 ql = ld128_a2(u + 64 * n + 32 * m + 16 * hh);
        const uint4 qh = ld128_a2(u + 128 + 32 * n + 16 * hh);
        // scales[16] and d: bytes 192..209.
        const uintptr_t ta = reinterpret_cast<uintptr_t>(u + 192);
        const uint8_t* tb = reinterpret_cast<const uint8_t*>(ta & ~uintptr_t(3));
        const uint32_t ts = static_cast<uint32_t>(ta & 3u);
        const uint4 t = ld128_a4(tb);
        const uint32_t t4 = *reinterpret_cast<const uint32_t*>(tb + 16);
        const uint32_t sc0_3 = __builtin_amdgcn_alignbyte(t.y, t.x, ts);
        const uint32_t sc4_7 = __builtin_amdgcn_alignbyte(t.z, t.y, ts);
        const uint32_t sc8_11 = __builtin_amdgcn_alignbyte(t.w, t.z, ts);
        const uint32_t sc12_15 = __builtin_amdgcn_alignbyte(t4, t.w, ts);
        const uint32_t dbits = __builtin_amdgcn_alignbyte(t4, t4, ts) & 0xffffu;  // bytes 16..17 of the tail
        // Scale bytes used: index 8n + hh + 2m (low nibbles) and +4 (high).
        const uint32_t wlo = n ? sc8_11 : sc0_3;
        const uint32_t whi = n ? sc12_15 : sc4_7;
        const uint32_t sel = 8 * (hh + 2 * m);
        const int8_t sA = static_cast<int8_t>((wlo >> sel) & 0xffu);
        const int8_t sB = static_cast<int8_t>((whi >> sel) & 0xffu);
        const float d = half_lo(dbits);
        const uint32_t e0 = 128 * n + 32 * m + 16 * hh;
        const float* xa = x + e0;
        const float* xb = x + e0 + 64;
        const uint32_t shl = 4 - 2 * m;  // qh bits (2m, 2m+1) -> bits 4, 5
        const uint32_t shr = 2 * m;      // qh bits (2m+4, 2m+5) -> bits 4, 5
        float s0 = 0.0f, s1 = 0.0f;
        const uint32_t L[4] = {ql.x, ql.y, ql.z, ql.w};
        const uint32_t H[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (L[i] & 0x0f0f0f0fu) | ((H[i] << shl) & 0x30303030u);
            const uint32_t hi = ((L[i] >> 4) & 0x0f0f0f0fu) | ((H[i] >> shr) & 0x30303030u);
            s0 = dot4_u8(lo, ldx4(xa + 4 * i), s0);
            s1 = dot4_u8(hi, ldx4(xb + 4 * i), s1);
        }
        // value = d * sc * (q - 32)
        const float r0 = d * static_cast<float>(sA) * (s0 - 32.0f * xs16[e0 >> 4]);
        const float r1 = d * static_cast<float>(sB) * (s1 - 32.0f * xs16[(e0 + 64) >> 4]);
        return r0 + r1;
    }
};

// Q8_0: two 34-byte blocks {d, qs[32] int8} per unit. Lane c = (b, p) takes
// bytes [8p, 8p+8) of block b: elements 32b + 8p + i. Signed bytes are
// flipped to unsigned (q + 128) and the -128 sum is added once per 16-group
// by the even-p lane.
template <>
struct Unit<kQ8_0> {
    static constexpr uint32_t elems = 64;
    static constexpr uint32_t bytes = 68;
    __device__ static __forceinline__ float dot(const uint8_t* u, uint32_t c, const float* x,
                                                const float* xs16) {
        const uint32_t b = c >> 2, p = c & 3;
        const uint8_t* blk = u + 34 * b;
        const uint32_t dbits = load_u16_a2(blk);
        const uint2 q = load_u64_a2(blk + 2 + 8 * p);
        const uint32_t e0 = 32 * b + 8 * p;
        float s = 0.0f;
        s = dot4_u8(q.x ^ 0x80808080u, ldx4(x + e0), s);
        s = dot4_u8(q.y ^ 0x80808080u, ldx4(x + e0 + 4), s);
        if ((p & 1) == 0) s -= 128.0f * xs16[e0 >> 4];
        return half_lo(dbits) * s;
    }
};

// Q5_0: two 22-byte blocks {d, qh[4], qs[16]} per unit. Lane c = (b, p)
// takes qs bytes [4p, 4p+4) of block b: low nibbles are elements 32b+4p+i,
// high nibbles 32b+16+4p+i; the fifth bits come from qh (model.cpp:581-601).
template <>
struct Unit<kQ5_0> {
    static constexpr uint32_t elems = 64;
    static constexpr uint32_t bytes = 44;
    __device__ static __forceinline__ float dot(const uint8_t* u, uint32_t c, const float* x,
                                                const float* xs16) {
        const uint32_t b = c >> 2, p = c & 3;
        const uint8_t* blk = u + 22 * b;
        const uint32_t dbits = load_u16_a2(blk);
        const uint32_t qh = load_u32_a2(blk + 2);
        const uint32_t qs = load_u32_a2(blk + 6 + 4 * p);
        const uint32_t hlo = (qh >> (4 * p)) & 0xfu;
        const uint32_t hhi = (qh >> (16 + 4 * p)) & 0xfu;
        const uint32_t lo = (qs & 0x0f0f0f0fu) | (((hlo * 0x00204081u) & 0x01010101u) << 4);
        const uint32_t hi = ((qs >> 4) & 0x0f0f0f0fu) | (((hhi * 0x00204081u) & 0x01010101u) << 4);
        const uint32_t e0 = 32 * b + 4 * p;
        float s = 0.0f;
        s = dot4_u8(lo, ldx4(x + e0), s);
        s = dot4_u8(hi, ldx4(x + e0 + 16), s);
        if (p == 0) s -= 16.0f * (xs16[(32 * b) >> 4] + xs16[(32 * b + 16) >> 4]);
        return half_lo(dbits) * s;
    }
};

// F32: 256 values (1024 bytes) per unit; lane c takes values [32c, 32c+32).
template <>
struct Unit<kF32> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 1024;
    __device__ static __forceinline__ float dot(const uint8_t* u, uint32_t c, const float* x,
                                                const float*) {
        const float* w = reinterpret_cast<const float*>(u) + 32 * c;
        const float* xv = x + 32 * c;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 a = ldx4(w + 4 * i);
            const float4 b = ldx4(xv + 4 * i);
            s = fmaf(a.x, b.x, s);
            s = fmaf(a.y, b.y, s);
            s = fmaf(a.z, b.z, s);
            s = fmaf(a.w, b.w, s);
        }
        return s;
    }
};

// F16: 256 values (512 bytes) per unit; lane c takes values [32c, 32c+32).
template <>
struct Unit<kF16> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 512;
    __device__ static __forceinline__ float dot(const uint8_t* u, uint32_t c, const float* x,
                                                const float*) {
        const uint8_t* w = u + 64 * c;
        const float* xv = x + 32 * c;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 h = ld128_a4(w + 16 * i);
            const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                s = fmaf(half_lo(hw[k]), xv[8 * i + 2 * k], s);
                s = fmaf(half_hi(hw[k]), xv[8 * i + 2 * k + 1], s);
            }
        }
        return s;
    }
};

__device__ __forceinline__ float octet_sum(float v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    return v;
}

// Sign-branched SiLU gate as in the reference SwiGLU (cpu_llm.cpp:188-202).
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float sig = g >= 0.0f ? 1.0f / (1.0f + expf(-g)) : expf(g) / (1.0f + expf(g));
    return g * sig * u;
}

// MODE 0: y = W x (+ bias) (+ residual).
// MODE 1: y = silu(W x) * (W2 x) over RB row pairs; when RB == 16 the block
//         also writes the per-16 sum of its outputs (the xs16 entry the next
//         GEMV consumes).
template <uint32_t T, int RB, int MODE>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                                                   size_t row_bytes, const float* __restrict__ x,
                                                   const float* __restrict__ xs16, const float* __restrict__ bias,
                                                   const float* __restrict__ residual, float* __restrict__ y,
                                                   float* __restrict__ ys16, uint32_t n, uint32_t units) {
    using U = Unit<T>;
    constexpr int VR = MODE == 1 ? 2 * RB : RB;  // virtual rows per block
    constexpr int OPR = 32 / VR;                  // octets per virtual row
    static_assert(OPR >= 1 && 32 % VR == 0, "rows per block must divide 32");
    const uint32_t tid = threadIdx.x;
    const uint32_t o = tid >> 3, c = tid & 7;
    const uint32_t vrow = o % VR, slot = o / VR;
    const uint32_t row = blockIdx.x * RB + (vrow % RB);
    const uint8_t* mat = (MODE == 1 && vrow >= RB) ? w2 : w;
    float acc = 0.0f;
    if (row < n) {
        const uint8_t* wr = mat + static_cast<size_t>(row) * row_bytes;
#pragma unroll 2
        for (uint32_t u = slot; u < units; u += OPR) {
            acc += U::dot(wr + static_cast<size_t>(u) * U::bytes, c, x + u * U::elems,
                          xs16 + u * (U::elems / 16));
        }
    }
    acc = octet_sum(acc);
    __shared__ float part[32];
    if (c == 0) part[o] = acc;
    __syncthreads();
    if (tid < static_cast<uint32_t>(RB)) {
        const uint32_t r = blockIdx.x * RB + tid;
        float s = 0.0f;
#pragma unroll
        for (int sl = 0; sl < OPR; ++sl) s += part[sl * VR + tid];
        float out = 0.0f;
        if (MODE == 0) {
            if (r < n) {
                if (bias) s += bias[r];
                if (residual) s += residual[r];
                y[r] = s;
            }
        } else {
            float g2 = 0.0f;
#pragma unroll
            for (int sl = 0; sl < OPR; ++sl) g2 += part[sl * VR + RB + tid];
            if (r < n) {
                out = silu_mul(s, g2);
                y[r] = out;
            }
            if (RB == 16 && ys16) {
                float t = out;
                t += __shfl_xor(t, 1);
                t += __shfl_xor(t, 2);
                t += __shfl_xor(t, 4);
                t += __shfl_xor(t, 8);
                if (tid == 0 && r < n) ys16[blockIdx.x] = t;
            }
        }
    }
}

// xs16[i] = sum of x[16 i .. 16 i + 15].
__global__ void prep_sums_kernel(const float* __restrict__ x, float* __restrict__ xs16, uint32_t groups) {
    const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    const float4* p = reinterpret_cast<const float4*>(x + 16 * g);
    const float4 a = p[0], b = p[1], c = p[2], d = p[3];
    xs16[g] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) + ((c.x + c.y) + (c.z + c.w)) +
              ((d.x + d.y) + (d.z + d.w));
}

template <uint32_t T, int MODE>
int launch_typed(int rb, const void* w, const void* w2, size_t row_bytes, const float* x, const float* xs16,
                 const float* bias, const float* residual, float* y, float* ys16, uint32_t n, uint32_t units,
                 hipStream_t stream) {
    const auto* wp = static_cast<const uint8_t*>(w);
    const auto* wp2 = static_cast<const uint8_t*>(w2);
    const dim3 block(256);
    const dim3 grid((n + rb - 1) / rb);
    switch (rb) {
#define HIPLLM_GEMV_CASE(R)                                                                                 \
    case R:                                                                                                 \
        hipLaunchKernelGGL((gemv_kernel<T, R, MODE>), grid, block, 0, stream, wp, wp2, row_bytes, x, xs16, \
                           bias, residual, y, ys16, n, units);                                              \
        break;
        HIPLLM_GEMV_CASE(2)
        HIPLLM_GEMV_CASE(4)
        HIPLLM_GEMV_CASE(8)
        HIPLLM_GEMV_CASE(16)
#undef HIPLLM_GEMV_CASE
    case 32:
        if (MODE == 1) return kInvalidArgument;
        hipLaunchKernelGGL((gemv_kernel<T, 32, 0>), grid, block, 0, stream, wp, wp2, row_bytes, x, xs16, bias,
                           residual, y, ys16, n, units);
        break;
    default:
        return kInvalidArgument;
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

uint32_t unit_elems(uint32_t type) {
    switch (type) {
    case kQ4_K: case kQ6_K: case kF32: case kF16: return 256;
    case kQ8_0: case kQ5_0: return 64;
    default: return 0;
    }
}

}  // namespace

// Rows per block: as many as keeps >= ~4 blocks per CU on a 256-CU part, so
// wave instructions share activation loads across rows without starving the
// machine; MODE 1 keeps 16 so the block can emit the next xs16 entry.
int gemv_default_rows(uint32_t n, uint32_t units) {
    const uint32_t target_blocks = 1024;
    for (int rb : {32, 16, 8, 4}) {
        if (n / static_cast<uint32_t>(rb) >= target_blocks && units >= static_cast<uint32_t>(32 / rb)) return rb;
    }
    if (units >= 16 && n <= 4096) return 2;
    return 4;
}

int launch_prep_sums(const float* x, float* xs16, size_t k, hipStream_t stream) {
    if (!x || !xs16 || k == 0 || k % 16 != 0) return kInvalidArgument;
    const uint32_t groups = static_cast<uint32_t>(k / 16);
    hipLaunchKernelGGL(prep_sums_kernel, dim3((groups + 255) / 256), dim3(256), 0, stream, x, xs16, groups);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

// GEMV over pre-computed xs16. rows_per_block 0 selects the default.
int launch_gemv_prepped(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* xs16,
                        const float* bias, const float* residual, float* y, size_t n, size_t k,
                        int rows_per_block, hipStream_t stream) {
    const uint32_t ue = unit_elems(type);
    if (!w || !x || !xs16 || !y || n == 0 || k == 0 || ue == 0) return kInvalidArgument;
    if (k % ue != 0) return kInvalidArgument;
    if (row_bytes < k / block_elems(type) * block_bytes(type)) return kInvalidArgument;
    if (type == kQ4_K && (row_bytes % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 16 != 0)) return kInvalidArgument;
    if ((type == kF32 || type == kF16) && (row_bytes % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 16 != 0)) {
        return kInvalidArgument;
    }
    if (reinterpret_cast<uintptr_t>(w) % 2 != 0 || row_bytes % 2 != 0) return kInvalidArgument;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return kInvalidArgument;
    if (n > 0x7fffffffu || k > 0x7fffffffu) return kLengthError;
    const uint32_t units = static_cast<uint32_t>(k / ue);
    const int rb = rows_per_block ? rows_per_block : gemv_default_rows(static_cast<uint32_t>(n), units);
    const uint32_t nn = static_cast<uint32_t>(n);
    switch (type) {
    case kQ4_K: return launch_typed<kQ4_K, 0>(rb, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    case kQ6_K: return launch_typed<kQ6_K, 0>(rb, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    case kQ8_0: return launch_typed<kQ8_0, 0>(rb, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    case kQ5_0: return launch_typed<kQ5_0, 0>(rb, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    case kF32: return launch_typed<kF32, 0>(rb, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    case kF16: return launch_typed<kF16, 0>(rb, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    default: return kInvalidArgument;
    }
}

// Fused gate/up GEMV + SwiGLU: y = silu(Wg x) * (Wu x); ys16 (optional,
// n % 16 == 0) receives per-16 sums of y for the down projection.
int launch_gemv_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                       const float* xs16, float* y, float* ys16, size_t n, size_t k, hipStream_t stream) {
    const uint32_t ue = unit_elems(type);
    if (!wg || !wu || !x || !xs16 || !y || n == 0 || k == 0 || ue == 0 || k % ue != 0) return kInvalidArgument;
    if (row_bytes < k / block_elems(type) * block_bytes(type)) return kInvalidArgument;
    if (type == kQ4_K && (row_bytes % 16 != 0 || reinterpret_cast<uintptr_t>(wg) % 16 != 0 ||
                          reinterpret_cast<uintptr_t>(wu) % 16 != 0)) {
        return kInvalidArgument;
    }
    if (ys16 && n % 16 != 0) return kInvalidArgument;
    if (n > 0x7fffffffu || k > 0x7fffffffu) return kLengthError;
    const uint32_t units = static_cast<uint32_t>(k / ue);
    const uint32_t nn = static_cast<uint32_t>(n);
    switch (type) {
    case kQ4_K: return launch_typed<kQ4_K, 1>(16, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    case kQ6_K: return launch_typed<kQ6_K, 1>(16, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    case kQ8_0: return launch_typed<kQ8_0, 1>(16, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    case kQ5_0: return launch_typed<kQ5_0, 1>(16, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    case kF32: return launch_typed<kF32, 1>(16, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    case kF16: return launch_typed<kF16, 1>(16, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    default: return kInvalidArgument;
    }
}

}  // namespace hipllm
