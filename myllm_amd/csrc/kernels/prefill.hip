// Prefill matmul Y[M,N] = X[M,K] W[N,K]^T (+ bias[N]) (+ residual[M,N]) on
// CDNA4 fp16 MFMA with FP32 accumulation, weights in native GGUF block layout.
//
// Replaces the reference's one-thread-per-output quantized GEMMs
// (metal_gemm_{q5_0,q8_0,q4_k,q6_k}_f32, metal_llm.metal:621-704; host
// encode_matrix_product, metal_llm.mm:1782-1889) and CPULLM's gemmt/gemmtb
// (cpu_llm.cpp:591-607, 631-653), which re-decode a weight row per output.
//
// Design:
// * Operands are fp16 (11 significant bits, 8x finer than bf16's 8, at the
//   same MFMA rate on gfx950). X is converted once per row
//   (to_f16_kernel): the row is scaled by a power of two that brings its
//   largest magnitude to [2^13, 2^14), rounded to nearest even, and the
//   inverse power of two is kept per row (xscale) and applied to the FP32
//   accumulator in the epilogue, so neither range nor precision depends on
//   the row's magnitude and the scaling itself is exact.
// * A block is 4 waves. Block tile = (4 * 32 * NSUB) weight rows x (32 * MSUB)
//   X rows; every wave owns 32 * NSUB weight rows and all 32 * MSUB X rows.
// * K advances in steps of 128. Each step, the X tile (fp16) is staged in LDS
//   (double-buffered, one barrier per step) and every wave dequantizes its own
//   weight rows straight from HBM into MFMA operand registers, so weights are
//   read once per X-row tile and never pass through LDS.
// * v_mfma_f32_32x32x16_f16: operand lane l holds row (l % 32) and eight
//   consecutive k. Inside a 128-k step, slice s (0..7) gives lane half
//   h = l / 32 the k range 64 G + 32 hi + 16 h + 8 p + [0, 8) with G = s >> 2,
//   hi = (s >> 1) & 1, p = s & 1. X and W use the same map, so each MFMA sums
//   over a permutation of its 16 k. This map lines up with the GGUF layouts:
//   Q4_K's low/high nibbles (hi), Q6_K's quarters, Q8_0/Q5_0's 32-blocks.
// * Dequantized values are computed in FP32 from the reference dequantizer's
//   scales and offsets (model.cpp:581-683), one fused multiply-add per value,
//   and rounded once to fp16 (F16 weights are used as stored). Weight values
//   must lie inside the fp16 range (|w| < 65504), as every GGUF block scale
//   of a trained or synthetic model does by far.
#include "common.h"
#include "norm.h"

namespace hipllm {

typedef _Float16 hx8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

namespace {

constexpr int kStepK = 128;
constexpr int kLdsRow = kStepK + 8;  // fp16 per LDS row: 272 bytes, spreads rows over banks

__device__ __forceinline__ uint4 g_ld128_a4(const uint8_t* p) {
    const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes from a 2-byte-aligned address (reads the enclosing dwords).
__device__ __forceinline__ uint4 g_ld128_a2(const uint8_t* p) {
    const uint32_t s = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint8_t* base = p - s;
    const uint4 v = g_ld128_a4(base);
    const uint32_t e = *reinterpret_cast<const uint32_t*>(base + 16);
    return make_uint4(__builtin_amdgcn_alignbyte(v.y, v.x, s), __builtin_amdgcn_alignbyte(v.z, v.y, s),
                      __builtin_amdgcn_alignbyte(v.w, v.z, s), __builtin_amdgcn_alignbyte(e, v.w, s));
}

__device__ __forceinline__ uint32_t g_ld32_a2(const uint8_t* p) {
    const uint32_t s = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p - s);
    return __builtin_amdgcn_alignbyte(q[1], q[0], s);
}

__device__ __forceinline__ float f16_bits(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits & 0xffffu)));
}

// fp16 pairs and fragments built from dwords: v_cvt_pk_f16_f32 rounds two
// floats to nearest even in one instruction, and the fragment is four such
// dwords, so no byte shuffles are needed to assemble it.
typedef _Float16 hx2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
    const f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, hx2));
}

// Hides a value's known bits from the optimizer, so that byte k of a masked
// dword converts with one v_cvt_f32_ubyte{k} instead of a shift, a mask and
// a byte-0 convert.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}

// Eight values v[i] = a * byte_i - b over the 8 bytes of (w0, w1), one fused
// multiply-add each, rounded to fp16. Where b is a power-of-two multiple of a
// (Q6_K's 32 a, Q8_0's 128 d) the result equals the reference's a * (q - c)
// exactly; for Q4_K / Q5_0 it differs from the reference's rounded product
// minus offset by at most one FP32 rounding, far below the fp16 rounding that
// follows.
__device__ __forceinline__ hx8 affine8(uint32_t w0, uint32_t w1, float a, float b) {
    w0 = opaque(w0);
    w1 = opaque(w1);
    const u32x4 u = {pack_h2(__builtin_fmaf(a, ubyte0(w0), -b), __builtin_fmaf(a, ubyte1(w0), -b)),
                     pack_h2(__builtin_fmaf(a, ubyte2(w0), -b), __builtin_fmaf(a, ubyte3(w0), -b)),
                     pack_h2(__builtin_fmaf(a, ubyte0(w1), -b), __builtin_fmaf(a, ubyte1(w1), -b)),
                     pack_h2(__builtin_fmaf(a, ubyte2(w1), -b), __builtin_fmaf(a, ubyte3(w1), -b))};
    return __builtin_bit_cast(hx8, u);
}

// Eight values v[i] = a * (byte_i - 32) (Q6_K) as a * byte_i - 32 a.
__device__ __forceinline__ hx8 q6_8(uint32_t w0, uint32_t w1, float a) {
    return affine8(w0, w1, a, 32.0f * a);
}

// Eight signed bytes times d (Q8_0: v = q * d) as d * (q + 128) - 128 d.
__device__ __forceinline__ hx8 q8_8(uint32_t w0, uint32_t w1, float d) {
    return affine8(w0 ^ 0x80808080u, w1 ^ 0x80808080u, d, 128.0f * d);
}
// Per-type weight fragments. Raw holds the bytes one lane needs for one
// 128-k step of one weight row; load() issues the global loads, slice<s>()
// turns them into the eight hx8 operands (slice order above).
template <uint32_t T>
struct WTile;

// Q4_K (144-byte super-blocks, model.cpp:616-644). A 128-k step is half a
// super-block: 64-groups j0 = 2 * (step % 2) and j0 + 1. Lane half h reads qs
// bytes [32 j + 16 h, +16) of each group: low nibbles are sub-block 2j,
// elements 16 h + [0, 16), high nibbles sub-block 2j + 1.
template <>
struct WTile<kQ4_K> {
    struct Raw {
        uint4 head;
        uint4 q[2];
    };
    __device__ static __forceinline__ Raw load(const uint8_t* row, uint32_t kb, uint32_t h) {
        const uint8_t* blk = row + (kb / 256) * 144;
        const uint32_t j0 = (kb % 256) / 64;
        Raw r;
        r.head = g_ld128_a4(blk);
        r.q[0] = g_ld128_a4(blk + 16 + 32 * j0 + 16 * h);
        r.q[1] = g_ld128_a4(blk + 16 + 32 * (j0 + 1) + 16 * h);
        return r;
    }
    // Slice s = 4 G + j: G picks the 64-group, j = 0, 1 the low nibbles of
    // qs dwords (x, y) / (z, w), j = 2, 3 the high nibbles.
    template <int S>
    __device__ static __forceinline__ hx8 slice(const Raw& r, uint32_t kb, uint32_t) {
        constexpr int G = S >> 2, J = S & 3;
        const uint32_t j0 = (kb % 256) / 64;
        const float d = f16_bits(r.head.x);
        const float dmin = f16_bits(r.head.x >> 16);
        // get_scale_min_k4 (model.cpp:524-537) for the four sub-blocks 2 j0 .. 2 j0 + 3,
        // both halves computed and selected with a mask (no branch).
        const uint32_t S0 = r.head.y & 0x3f3f3f3fu, M0 = r.head.z & 0x3f3f3f3fu;
        const uint32_t S1 = (r.head.w & 0x0f0f0f0fu) | ((r.head.y >> 2) & 0x30303030u);
        const uint32_t M1 = ((r.head.w >> 4) & 0x0f0f0f0fu) | ((r.head.z >> 2) & 0x30303030u);
        const uint32_t hi_half = 0u - static_cast<uint32_t>(j0 != 0);
        const uint32_t Sc = (S0 & ~hi_half) | (S1 & hi_half);
        const uint32_t Mn = (M0 & ~hi_half) | (M1 & hi_half);
        constexpr int sh = 16 * G + (J >= 2 ? 8 : 0);
        const float d1 = d * static_cast<float>((Sc >> sh) & 0xffu);
        const float m1 = dmin * static_cast<float>((Mn >> sh) & 0xffu);
        const uint4 q = r.q[G];
        const uint32_t a0 = (J & 1) ? q.z : q.x, a1 = (J & 1) ? q.w : q.y;
        constexpr int ns = J >= 2 ? 4 : 0;
        return affine8((a0 >> ns) & 0x0f0f0f0fu, (a1 >> ns) & 0x0f0f0f0fu, d1, m1);
    }
};

// Q6_K (210-byte super-blocks, model.cpp:646-683). A 128-k step is the half
// n6 = step % 2; slice (G, hi) is quarter 2 G + hi. Lane half h needs
// l = 16 h + [0, 16): ql bytes 64 n6 + 32 hi + l (low nibble for G = 0, high
// for G = 1), qh byte 32 n6 + l shifted by 2 * quarter, scale
// sc[8 n6 + h + 2 * quarter].
template <>
struct WTile<kQ6_K> {
    struct Raw {
        uint4 ql[2];
        uint4 qh;
        uint32_t sc;  // scales 8 n6 + h + {0, 2, 4, 6}
        uint32_t d;
    };
    __device__ static __forceinline__ Raw load(const uint8_t* row, uint32_t kb, uint32_t h) {
        const uint8_t* blk = row + (kb / 256) * 210;
        const uint32_t n6 = (kb % 256) / 128;
        Raw r;
        r.ql[0] = g_ld128_a2(blk + 64 * n6 + 16 * h);
        r.ql[1] = g_ld128_a2(blk + 64 * n6 + 32 + 16 * h);
        r.qh = g_ld128_a2(blk + 128 + 32 * n6 + 16 * h);
        const uint32_t lo = g_ld32_a2(blk + 192 + 8 * n6);      // scales 8 n6 + 0..3
        const uint32_t hi = g_ld32_a2(blk + 192 + 8 * n6 + 4);  // scales 8 n6 + 4..7
        // bytes h, h + 2 of lo and h, h + 2 of hi -> quarters 0, 1, 2, 3
        const uint32_t sh = 8 * h;
        r.sc = ((lo >> sh) & 0xffu) | (((lo >> (sh + 16)) & 0xffu) << 8) | (((hi >> sh) & 0xffu) << 16) |
               (((hi >> (sh + 16)) & 0xffu) << 24);
        r.d = g_ld32_a2(blk + 208) & 0xffffu;
        return r;
    }
    // Slice s = 4 G + 2 hi + j: quarter 2 G + hi, qs dwords (x, y) or (z, w).
    template <int S>
    __device__ static __forceinline__ hx8 slice(const Raw& r, uint32_t, uint32_t) {
        constexpr int G = S >> 2, HI = (S >> 1) & 1, J = S & 1;
        constexpr int quarter = 2 * G + HI;
        const float d = f16_bits(r.d);
        const int8_t scb = static_cast<int8_t>((r.sc >> (8 * quarter)) & 0xffu);
        const float a = d * static_cast<float>(scb);
        const uint4 l = r.ql[HI];
        const uint32_t L0 = J ? l.z : l.x, L1 = J ? l.w : l.y;
        const uint32_t H0 = J ? r.qh.z : r.qh.x, H1 = J ? r.qh.w : r.qh.y;
        constexpr int ns = G == 0 ? 0 : 4;
        const uint32_t v0 = ((L0 >> ns) & 0x0f0f0f0fu) | (((H0 >> (2 * quarter)) & 0x03030303u) << 4);
        const uint32_t v1 = ((L1 >> ns) & 0x0f0f0f0fu) | (((H1 >> (2 * quarter)) & 0x03030303u) << 4);
        return q6_8(v0, v1, a);
    }
};

// Q8_0 (34-byte blocks, model.cpp:603-614): slice (G, hi) is block 4 s' with
// s' = 2 G + hi of the step; lane half h takes bytes 16 h + [0, 16).
template <>
struct WTile<kQ8_0> {
    struct Raw {
        uint4 q[4];
        uint32_t d[4];
    };
    __device__ static __forceinline__ Raw load(const uint8_t* row, uint32_t kb, uint32_t h) {
        const uint8_t* blk = row + (kb / 32) * 34;
        Raw r;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            r.q[b] = g_ld128_a2(blk + 34 * b + 2 + 16 * h);
            r.d[b] = g_ld32_a2(blk + 34 * b) & 0xffffu;
        }
        return r;
    }
    template <int S>
    __device__ static __forceinline__ hx8 slice(const Raw& r, uint32_t, uint32_t) {
        constexpr int B = S >> 1, J = S & 1;
        const float d = f16_bits(r.d[B]);
        return J ? q8_8(r.q[B].z, r.q[B].w, d) : q8_8(r.q[B].x, r.q[B].y, d);
    }
};

// Q5_0 (22-byte blocks, model.cpp:581-601): slice (G, hi) is block 2 G + hi;
// lane half h takes elements 16 h + [0, 16): the low (h = 0) or high (h = 1)
// nibbles of qs[0..16), fifth bits qh >> (16 h + i); v = q d - 16 d.
template <>
struct WTile<kQ5_0> {
    struct Raw {
        uint4 q[4];
        uint32_t qh[4];
        uint32_t d[4];
    };
    __device__ static __forceinline__ Raw load(const uint8_t* row, uint32_t kb, uint32_t) {
        const uint8_t* blk = row + (kb / 32) * 22;
        Raw r;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            r.d[b] = g_ld32_a2(blk + 22 * b) & 0xffffu;
            r.qh[b] = g_ld32_a2(blk + 22 * b + 2);
            r.q[b] = g_ld128_a2(blk + 22 * b + 6);
        }
        return r;
    }
    template <int S>
    __device__ static __forceinline__ hx8 slice(const Raw& r, uint32_t, uint32_t h) {
        constexpr int B = S >> 1, J = S & 1;
        const float d = f16_bits(r.d[B]);
        const float m = 16.0f * d;
        const uint32_t bits = r.qh[B] >> (16 * h);  // fifth bits of elements 16 h + i
        const uint32_t Q[4] = {r.q[B].x, r.q[B].y, r.q[B].z, r.q[B].w};
        uint32_t v[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int i = 2 * J + t;
            const uint32_t nib = h == 0 ? (Q[i] & 0x0f0f0f0fu) : ((Q[i] >> 4) & 0x0f0f0f0fu);
            const uint32_t hb = (bits >> (4 * i)) & 0xfu;
            v[t] = nib | (((hb * 0x00204081u) & 0x01010101u) << 4);
        }
        return affine8(v[0], v[1], d, m);
    }
};

// F32 weights: slice s covers k = 64 G + 32 hi + 16 h + 8 p + [0, 8).
template <>
struct WTile<kF32> {
    struct Raw {
        uint4 v[16];
    };
    __device__ static __forceinline__ Raw load(const uint8_t* row, uint32_t kb, uint32_t h) {
        const uint8_t* p = row + 4 * static_cast<size_t>(kb);
        Raw r;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint32_t k0 = 64 * (s >> 2) + 32 * ((s >> 1) & 1) + 16 * h + 8 * (s & 1);
            r.v[2 * s] = g_ld128_a4(p + 4 * k0);
            r.v[2 * s + 1] = g_ld128_a4(p + 4 * k0 + 16);
        }
        return r;
    }
    template <int S>
    __device__ static __forceinline__ hx8 slice(const Raw& r, uint32_t, uint32_t) {
        const uint4 a = r.v[2 * S], b = r.v[2 * S + 1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        hx8 f;
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = static_cast<_Float16>(__uint_as_float(w[i]));
        return f;
    }
};

// F16 weights.
template <>
struct WTile<kF16> {
    struct Raw {
        uint4 v[8];
    };
    __device__ static __forceinline__ Raw load(const uint8_t* row, uint32_t kb, uint32_t h) {
        const uint8_t* p = row + 2 * static_cast<size_t>(kb);
        Raw r;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint32_t k0 = 64 * (s >> 2) + 32 * ((s >> 1) & 1) + 16 * h + 8 * (s & 1);
            r.v[s] = g_ld128_a4(p + 2 * k0);
        }
        return r;
    }
    // The stored halves are the operands themselves.
    template <int S>
    __device__ static __forceinline__ hx8 slice(const Raw& r, uint32_t, uint32_t) {
        const u32x4 u = {r.v[S].x, r.v[S].y, r.v[S].z, r.v[S].w};
        return __builtin_bit_cast(hx8, u);
    }
};

// All eight slices of one lane's row fragment for one 128-k step.
template <uint32_t T>
__device__ __forceinline__ void wtile_frags(const typename WTile<T>::Raw& r, uint32_t kb, uint32_t h, hx8* f) {
    f[0] = WTile<T>::template slice<0>(r, kb, h);
    f[1] = WTile<T>::template slice<1>(r, kb, h);
    f[2] = WTile<T>::template slice<2>(r, kb, h);
    f[3] = WTile<T>::template slice<3>(r, kb, h);
    f[4] = WTile<T>::template slice<4>(r, kb, h);
    f[5] = WTile<T>::template slice<5>(r, kb, h);
    f[6] = WTile<T>::template slice<6>(r, kb, h);
    f[7] = WTile<T>::template slice<7>(r, kb, h);
}

// Block -> (weight-row tile, X-row tile), XCD-aware. Workgroups of one
// dispatch go to the 8 XCDs round-robin (block b to XCD b % 8), each XCD with
// its own L2. The linear block id is first renumbered so each XCD's blocks are
// consecutive, then walked in groups of kGroupM X tiles: consecutive blocks on
// one XCD share a weight tile (read into that XCD's L2 once per group) and the
// group's X rows stay in the same L2 across weight tiles.
constexpr uint32_t kXcds = 8, kGroupM = 4;
__device__ __forceinline__ void block_tile(uint32_t nbs, uint32_t mbs, uint32_t& nb, uint32_t& mb) {
    const uint32_t total = nbs * mbs, b = blockIdx.x;
    const uint32_t per = total / kXcds, rem = total % kXcds, x = b % kXcds;
    const uint32_t id = x * per + min(x, rem) + b / kXcds;
    const uint32_t span = kGroupM * nbs;
    const uint32_t first = id / span * kGroupM;
    const uint32_t gsize = min(mbs - first, kGroupM);
    const uint32_t in = id % span;
    mb = first + in % gsize;
    nb = in / gsize;
}

// Gathered form (routed expert products): block (weight tile x, group y)
// multiplies the rows of expert group y (launch_route_groups: at most 64
// routed vectors of one expert) by that expert's weights, gathering each
// vector's X row (row j / routes of xb, or row j when x_routed) and writing
// row j of y. Groups past *ngroups exit at once.
struct Gather {
    const int32_t* order = nullptr;
    const int32_t* groups = nullptr;
    const uint32_t* ngroups = nullptr;
    size_t expert_stride = 0;
    uint32_t routes = 1;
    uint32_t x_routed = 0;
};

template <uint32_t T, int NSUB, int MSUB, bool GATHER = false>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const uint8_t* __restrict__ w, size_t row_bytes,
                                                        const _Float16* __restrict__ xb,
                                                        const float* __restrict__ xscale,
                                                        const float* __restrict__ bias,
                                                        const float* __restrict__ residual, float* __restrict__ y,
                                                        uint32_t m, uint32_t n, uint32_t k, uint32_t ldy,
                                                        uint32_t steps_per_split, const Gather gather = Gather()) {
    using WT = WTile<T>;
    constexpr int BM = 32 * MSUB;
    constexpr int WN = 32 * NSUB;
    constexpr int BN = 4 * WN;
    constexpr int kLoads = BM * (kStepK / 8) / 256;  // 16-byte X loads per thread per step
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][BM * kLdsRow];

    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6, lane = tid & 63;
    const uint32_t lr = lane & 31, h = lane >> 5;
    uint32_t nb, mb;
    uint32_t gfirst = 0;  // GATHER: the group's first index into gather.order
    if constexpr (GATHER) {
        if (blockIdx.y >= *gather.ngroups) return;
        gfirst = static_cast<uint32_t>(gather.groups[2 * blockIdx.y]);
        const uint32_t packed = static_cast<uint32_t>(gather.groups[2 * blockIdx.y + 1]);
        w += static_cast<size_t>(packed & 0xffffu) * gather.expert_stride;
        m = packed >> 16;  // the group's rows
        nb = blockIdx.x;
        mb = 0;
    } else {
        block_tile((n + BN - 1) / BN, (m + BM - 1) / BM, nb, mb);
    }
    // GATHER: local row r is routed vector gather.order[gfirst + r].
    auto vec = [&](uint32_t r) { return static_cast<uint32_t>(gather.order[gfirst + r]); };
    const uint32_t m0 = mb * BM;
    const uint32_t n0 = nb * BN + wave * WN;

    const uint8_t* wrow[NSUB];
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns) {
        const uint32_t r = min(n0 + 32 * ns + lr, n - 1);  // rows past n read row n - 1, never stored
        wrow[ns] = w + static_cast<size_t>(r) * row_bytes;
    }

    // X tile loader: thread t moves 16 bytes (8 fp16) of row t / 16 + 16 i,
    // column chunk t % 16, for i < kLoads.
    uint4 xr[kLoads];
    auto load_x = [&](uint32_t kb) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const uint32_t row = tid / 16 + 16 * i;
            const uint32_t gm = m0 + row;
            if (gm < m) {
                size_t src = gm;
                if constexpr (GATHER) src = gather.x_routed ? vec(gm) : vec(gm) / gather.routes;
                xr[i] = *reinterpret_cast<const uint4*>(xb + src * k + kb + 8 * (tid % 16));
            } else {
                xr[i] = make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const uint32_t row = tid / 16 + 16 * i;
            *reinterpret_cast<uint4*>(&xs[buf][row * kLdsRow + 8 * (tid % 16)]) = xr[i];
        }
    };

    f32x16 acc[NSUB][MSUB];
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns)
#pragma unroll
        for (int ms = 0; ms < MSUB; ++ms)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[ns][ms][i] = 0.0f;

    // K split: block z covers steps [z * steps_per_split, ...) of the k / 128.
    const uint32_t kb0 = blockIdx.z * steps_per_split * kStepK;
    const uint32_t steps = min(steps_per_split, k / kStepK - blockIdx.z * steps_per_split);
    typename WT::Raw raw[NSUB];
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns) raw[ns] = WT::load(wrow[ns], kb0, h);
    load_x(kb0);
    store_x(0);
    __syncthreads();

    for (uint32_t st = 0; st < steps; ++st) {
        const uint32_t kb = kb0 + st * kStepK;
        const int buf = st & 1;
        hx8 bf[NSUB][8];
#pragma unroll
        for (int ns = 0; ns < NSUB; ++ns) wtile_frags<T>(raw[ns], kb, h, bf[ns]);
        if (st + 1 < steps) {
#pragma unroll
            for (int ns = 0; ns < NSUB; ++ns) raw[ns] = WT::load(wrow[ns], kb + kStepK, h);
            load_x(kb + kStepK);
        }
        const _Float16* xt = xs[buf];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint32_t kc = 64 * (s >> 2) + 32 * ((s >> 1) & 1) + 16 * h + 8 * (s & 1);
#pragma unroll
            for (int ms = 0; ms < MSUB; ++ms) {
                const hx8 a = *reinterpret_cast<const hx8*>(&xt[(32 * ms + lr) * kLdsRow + kc]);
#pragma unroll
                for (int ns = 0; ns < NSUB; ++ns) {
                    acc[ns][ms] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bf[ns][s], acc[ns][ms], 0, 0, 0);
                }
            }
        }
        if (st + 1 < steps) store_x(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: acc[ns][ms][4 g + r] = Y[m0 + 32 ms + 8 g + 4 h + r][n0 + 32 ns + lr]
    // in units of the row's X scale (exact power of two).
    // With a K split, y is the partial-sum buffer: split z stores its plane
    // z (m rows of ld ldy), and gemm_split_reduce_kernel adds the planes in
    // split order, so the result does not depend on which split ends first.
    const bool split = gridDim.z > 1;
#pragma unroll
    for (int ns = 0; ns < NSUB; ++ns) {
        const uint32_t col = n0 + 32 * ns + lr;
        if (col >= n) continue;
        const float b = (bias && !split) ? bias[col] : 0.0f;
#pragma unroll
        for (int ms = 0; ms < MSUB; ++ms) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t row = m0 + 32 * ms + 8 * g + 4 * h + r;
                    if (row < m) {
                        uint32_t src = row;
                        if constexpr (GATHER) src = gather.x_routed ? vec(row) : vec(row) / gather.routes;
                        const float a = acc[ns][ms][4 * g + r] * xscale[src];
                        const size_t o = static_cast<size_t>(GATHER ? vec(row) : row) * ldy + col;
                        if (split) {
                            y[static_cast<size_t>(blockIdx.z) * m * ldy + o] = a;
                        } else {
                            float v = a + b;
                            if (residual) v += residual[o];
                            y[o] = v;
                        }
                    }
                }
            }
        }
    }
}

// Shared-dequant form: the block's 128 weight rows are dequantized once per
// 128-k step into LDS, already in MFMA operand order, and every wave
// multiplies them into its own 32 * MT X rows, so each weight is converted
// once per 128 * MT X rows instead of once per 64.
// * Wave w dequantizes weight rows n0 + 32 w + [0, 32) (the WTile map: lane
//   (lr, h) gets the eight hx8 slices of row lr, half h) and stores slice
//   s at ws[buf][w][s][lane], 16 bytes per lane: a wave's reads and writes of
//   one slice are 1 KiB contiguous, free of bank conflicts.
// * X fragments are loaded from global memory straight into registers with
//   the same k map; waves own disjoint X rows, so each X element is read once
//   per block. Rows past m read row m - 1 and their outputs are dropped.
// * Software pipeline, one barrier per step: while the MFMAs of step st read
//   LDS buffer st % 2, the wave dequantizes step st + 1 (its bytes loaded one
//   step earlier) for the other buffer, and loads X of step st + 1 and the
//   weight bytes of step st + 2. The loop body is one basic block and a
//   scheduling pattern interleaves the dequant's VALU work with the MFMAs, so
//   the two run side by side on the SIMD. MT = 1 fits two waves per SIMD
//   (two blocks per CU); MT = 2 runs one.
template <uint32_t T, int MT>
__global__ __launch_bounds__(256, MT == 1 ? 2 : 1) void gemm_lds_kernel(const uint8_t* __restrict__ w, size_t row_bytes,
                                                          const _Float16* __restrict__ xb,
                                                          const float* __restrict__ xscale,
                                                          const float* __restrict__ bias,
                                                          const float* __restrict__ residual, float* __restrict__ y,
                                                          uint32_t m, uint32_t n, uint32_t k, uint32_t ldy,
                                                          uint32_t steps_per_split) {
    using WT = WTile<T>;
    __shared__ hx8 ws[2][4][8][64];

    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6, lane = tid & 63;
    const uint32_t lr = lane & 31, h = lane >> 5;
    uint32_t nb, mb;
    block_tile((n + 127) / 128, (m + 128 * MT - 1) / (128 * MT), nb, mb);
    const uint32_t n0 = nb * 128;
    const uint32_t mw = mb * (128 * MT) + wave * (32 * MT);  // this wave's first X row

    const uint8_t* wrow = w + static_cast<size_t>(min(n0 + 32 * wave + lr, n - 1)) * row_bytes;
    const _Float16* xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xrow[mt] = xb + static_cast<size_t>(min(mw + 32 * mt + lr, m - 1)) * k;
    auto load_x = [&](uint32_t kb, hx8 (&xa)[MT][8]) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const uint32_t kc = 64 * (s >> 2) + 32 * ((s >> 1) & 1) + 16 * h + 8 * (s & 1);
                xa[mt][s] = *reinterpret_cast<const hx8*>(xrow[mt] + kb + kc);
            }
        }
    };

    f32x16 acc[4][MT];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[nt][mt][i] = 0.0f;

    const uint32_t kb0 = blockIdx.z * steps_per_split * kStepK;
    const uint32_t steps = min(steps_per_split, k / kStepK - blockIdx.z * steps_per_split);
    const uint32_t klast = kb0 + (steps - 1) * kStepK;  // loads past the split re-read its last step
    hx8 xa[MT][8];
    load_x(kb0, xa);
    typename WT::Raw rawn;
    {
        const typename WT::Raw raw = WT::load(wrow, kb0, h);
        rawn = WT::load(wrow, min(kb0 + kStepK, klast), h);
        hx8 f[8];
        wtile_frags<T>(raw, kb0, h, f);
#pragma unroll
        for (int s = 0; s < 8; ++s) ws[0][wave][s][lane] = f[s];
    }
    __syncthreads();

    // One pipeline step. cur: this step's X fragments; nxt receives step
    // st + 1's. rn: step st + 1's weight bytes; r2 receives step st + 2's.
    auto body = [&](uint32_t st, hx8 (&cur)[MT][8], hx8 (&nxt)[MT][8], const typename WT::Raw& rn,
                    typename WT::Raw& r2) {
        const uint32_t kb = kb0 + st * kStepK;
        const int buf = st & 1;
        load_x(min(kb + kStepK, klast), nxt);
        r2 = WT::load(wrow, min(kb + 2 * kStepK, klast), h);
        // Slice by slice: the MFMAs of slice s on this step's tile, then
        // slice s of the next step's tile dequantized and stored, with the
        // next slice's weight fragments read ahead. A scheduling fence per
        // slice keeps each slice's VALU work beside its MFMAs.
        hx8 bcur[4], bnxt[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) bcur[nt] = ws[buf][nt][0][lane];
        auto slice_step = [&](auto sc) {
            constexpr int S = decltype(sc)::value;
            if constexpr (S < 7) {
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) bnxt[nt] = ws[buf][nt][S + 1][lane];
            }
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    acc[nt][mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[mt][S], bcur[nt], acc[nt][mt], 0, 0, 0);
                }
            }
            ws[buf ^ 1][wave][S][lane] = WT::template slice<S>(rn, kb + kStepK, h);  // unused after the last step
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (S < 7) {
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) bcur[nt] = bnxt[nt];
            }
        };
        slice_step(std::integral_constant<int, 0>{});
        slice_step(std::integral_constant<int, 1>{});
        slice_step(std::integral_constant<int, 2>{});
        slice_step(std::integral_constant<int, 3>{});
        slice_step(std::integral_constant<int, 4>{});
        slice_step(std::integral_constant<int, 5>{});
        slice_step(std::integral_constant<int, 6>{});
        slice_step(std::integral_constant<int, 7>{});
        __syncthreads();
    };
    // Two steps per iteration with the register sets swapped, so nothing is
    // copied between steps.
    hx8 xb2[MT][8];
    typename WT::Raw rawm;
    for (uint32_t st = 0; st < steps; st += 2) {
        body(st, xa, xb2, rawn, rawm);
        if (st + 1 < steps) body(st + 1, xb2, xa, rawm, rawn);
    }

    // Epilogue: acc[nt][mt][4 g + r] = Y[mw + 32 mt + 8 g + 4 h + r][n0 + 32 nt + lr];
    // with a K split, partial planes as in gemm_mfma_kernel.
    const bool split = gridDim.z > 1;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const uint32_t col = n0 + 32 * nt + lr;
        if (col >= n) continue;
        const float b = (bias && !split) ? bias[col] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t row = mw + 32 * mt + 8 * g + 4 * h + r;
                    if (row < m) {
                        const float a = acc[nt][mt][4 * g + r] * xscale[row];
                        const size_t o = static_cast<size_t>(row) * ldy + col;
                        if (split) {
                            y[static_cast<size_t>(blockIdx.z) * m * ldy + o] = a;
                        } else {
                            float v = a + b;
                            if (residual) v += residual[o];
                            y[o] = v;
                        }
                    }
                }
            }
        }
    }
}

// y[r, c] = (part[0][r, c] + part[1][r, c] + ... + part[splits - 1][r, c])
// + bias[c] + residual[r, c] (either may be absent), the partial planes
// (m x n, dense) added in split order: a K-split product gives the same bits
// on every run. The additions after the sum follow the unsplit epilogue.
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(const float* __restrict__ part, uint32_t splits,
                                                                const float* __restrict__ bias,
                                                                const float* residual, float* y, uint32_t m,
                                                                uint32_t n, uint32_t ldy) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t plane = static_cast<size_t>(m) * n;
    if (i >= plane) return;
    const uint32_t r = static_cast<uint32_t>(i / n), c = static_cast<uint32_t>(i % n);
    float a = part[i];
    for (uint32_t z = 1; z < splits; ++z) a += part[z * plane + i];
    float v = a + (bias ? bias[c] : 0.0f);
    const size_t o = static_cast<size_t>(r) * ldy + c;
    if (residual) v += residual[o];
    y[o] = v;
}

// Row r of x as fp16 operands: xh[r, c] = fp16(x[r, c] * 2^-e) (round to
// nearest even) and xscale[r] = 2^e, with e chosen so the row's largest
// magnitude lands in [2^13, 2^14): far from fp16 overflow (65504) and with
// the row's significant values in the normal range. Both scalings are exact
// powers of two (e is kept in [-126, 127], so 2^-e stays finite). NaN values
// are left out of the maximum and stay NaN; a row of zeros, or one holding
// an Inf, keeps e = 0 (the non-finite values then reach the output as they
// would in FP32). Block (r, c) converts values [2048 c, 2048 c + 2048) of
// row r, after reading the whole row for its maximum (every block of a row
// computes the same e).
constexpr uint32_t kF16Chunk = 2048;
__global__ __launch_bounds__(256) void to_f16_kernel(const float* __restrict__ x, size_t ldx,
                                                     _Float16* __restrict__ xh, float* __restrict__ xscale,
                                                     uint32_t k) {
    const uint32_t r = blockIdx.x;
    const float4* xr = reinterpret_cast<const float4*>(x + static_cast<size_t>(r) * ldx);
    const uint32_t k4 = k / 4;
    float mx = 0.0f;
    for (uint32_t i = threadIdx.x; i < k4; i += 256) {
        const float4 v = xr[i];
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    __shared__ float red[4];
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (mx > 0.0f && mx <= 3.402823466e38f) {
        frexpf(mx, &e);  // mx = f 2^e, f in [0.5, 1)
        e = max(-126, min(127, e - 14));
    }
    const float down = ldexpf(1.0f, -e);
    if (threadIdx.x == 0 && blockIdx.y == 0) xscale[r] = ldexpf(1.0f, e);
    _Float16* dst = xh + static_cast<size_t>(r) * k;
    const uint32_t end = min(k, (blockIdx.y + 1) * kF16Chunk) / 8;
    for (uint32_t i = blockIdx.y * (kF16Chunk / 8) + threadIdx.x; i < end; i += 256) {
        const float4 a = xr[2 * i], b = xr[2 * i + 1];
        const u32x4 u = {pack_h2(a.x * down, a.y * down), pack_h2(a.z * down, a.w * down),
                         pack_h2(b.x * down, b.y * down), pack_h2(b.z * down, b.w * down)};
        *reinterpret_cast<u32x4*>(dst + 8 * i) = u;
    }
}

// A row's RMSNorm and its fp16 operand form in one launch: the norm of
// rmsnorm_row_groups (norm receives the FP32 row, as the norm kernel writes
// it), then to_f16_kernel's conversion of that row, each thread converting
// the 16-value groups it normalised (its own writes, read back), the row's
// maximum reduced as there: the same bits as the two launches. One block
// of 256 threads per row; k % 16 == 0 and k <= 8192.
__global__ __launch_bounds__(256) void rmsnorm_f16_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                          float* __restrict__ norm, _Float16* __restrict__ xh,
                                                          float* __restrict__ xscale, uint32_t k, float eps) {
    const uint32_t r = blockIdx.x, tid = threadIdx.x, groups = k / 16;
    float* yr = norm + static_cast<size_t>(r) * k;
    rmsnorm_row_groups(x + static_cast<size_t>(r) * k, gamma, yr, nullptr, k, eps);
    float v[2][16];
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t g = tid + 256 * j;
        if (g < groups) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                v[j][i] = yr[16 * g + i];
                mx = fmaxf(mx, fabsf(v[j][i]));
            }
        }
    }
    __shared__ float red[4];
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (mx > 0.0f && mx <= 3.402823466e38f) {
        frexpf(mx, &e);  // mx = f 2^e, f in [0.5, 1)
        e = max(-126, min(127, e - 14));
    }
    const float down = ldexpf(1.0f, -e);
    if (tid == 0) xscale[r] = ldexpf(1.0f, e);
    _Float16* dst = xh + static_cast<size_t>(r) * k;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t g = tid + 256 * j;
        if (g < groups) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float* a = v[j] + 8 * h;
                const u32x4 u = {pack_h2(a[0] * down, a[1] * down), pack_h2(a[2] * down, a[3] * down),
                                 pack_h2(a[4] * down, a[5] * down), pack_h2(a[6] * down, a[7] * down)};
                *reinterpret_cast<u32x4*>(dst + 16 * g + 8 * h) = u;
            }
        }
    }
}

// A K split of `splits` planes of `per` 128-k steps each writes its partial
// sums to `part` (splits * m * n floats) and one reduce launch adds them.
void launch_split_reduce(const float* part, uint32_t splits, const float* bias, const float* residual, float* y,
                         uint32_t m, uint32_t n, uint32_t ldy, hipStream_t stream) {
    const size_t total = static_cast<size_t>(m) * n;
    HIPLLM_LAUNCH(gemm_split_reduce_kernel, dim3(static_cast<uint32_t>((total + 255) / 256)), dim3(256), 0, stream,
                  part, splits, bias, residual, y, m, n, ldy);
}

template <uint32_t T, int NSUB, int MSUB>
void launch_tile(const void* w, size_t row_bytes, const _Float16* xb, const float* xscale, const float* bias,
                 const float* residual, float* y, uint32_t m, uint32_t n, uint32_t k, uint32_t ldy, uint32_t splits,
                 uint32_t per, float* part, hipStream_t stream, bool reduce = true) {
    constexpr uint32_t BN = 4 * 32 * NSUB, BM = 32 * MSUB;
    const dim3 grid(((n + BN - 1) / BN) * ((m + BM - 1) / BM), 1, splits);
    if (splits > 1) {
        HIPLLM_LAUNCH((gemm_mfma_kernel<T, NSUB, MSUB>), grid, dim3(256), 0, stream, static_cast<const uint8_t*>(w),
                      row_bytes, xb, xscale, nullptr, nullptr, part, m, n, k, n, per);
        if (reduce) launch_split_reduce(part, splits, bias, residual, y, m, n, ldy, stream);
    } else {
        HIPLLM_LAUNCH((gemm_mfma_kernel<T, NSUB, MSUB>), grid, dim3(256), 0, stream, static_cast<const uint8_t*>(w),
                      row_bytes, xb, xscale, bias, residual, y, m, n, k, ldy, per);
    }
}

// The gathered expert products: tile 1 (64 rows x 128 weight rows per
// block, matching groups of at most 64 vectors), no K split.
template <uint32_t T>
void launch_gather(const void* w, size_t row_bytes, const _Float16* xb, const float* xscale, float* y, uint32_t n,
                   uint32_t k, uint32_t ldy, uint32_t max_groups, const Gather& g, hipStream_t stream) {
    constexpr uint32_t BN = 4 * 32;
    const dim3 grid((n + BN - 1) / BN, max_groups, 1);
    HIPLLM_LAUNCH((gemm_mfma_kernel<T, 1, 2, true>), grid, dim3(256), 0, stream, static_cast<const uint8_t*>(w),
                       row_bytes, xb, xscale, nullptr, nullptr, y, 0u, n, k, ldy, k / kStepK, g);
}

template <uint32_t T, int MT>
void launch_lds(const void* w, size_t row_bytes, const _Float16* xb, const float* xscale, const float* bias,
                const float* residual, float* y, uint32_t m, uint32_t n, uint32_t k, uint32_t ldy, uint32_t splits,
                uint32_t per, float* part, hipStream_t stream, bool reduce = true) {
    constexpr uint32_t BN = 128, BM = 128 * MT;
    const dim3 grid(((n + BN - 1) / BN) * ((m + BM - 1) / BM), 1, splits);
    if (splits > 1) {
        HIPLLM_LAUNCH((gemm_lds_kernel<T, MT>), grid, dim3(256), 0, stream, static_cast<const uint8_t*>(w), row_bytes,
                      xb, xscale, nullptr, nullptr, part, m, n, k, n, per);
        if (reduce) launch_split_reduce(part, splits, bias, residual, y, m, n, ldy, stream);
    } else {
        HIPLLM_LAUNCH((gemm_lds_kernel<T, MT>), grid, dim3(256), 0, stream, static_cast<const uint8_t*>(w), row_bytes,
                      xb, xscale, bias, residual, y, m, n, k, ldy, per);
    }
}

template <uint32_t T>
int launch_typed(int tile, const void* w, size_t row_bytes, const _Float16* xb, const float* xscale,
                 const float* bias, const float* residual, float* y, uint32_t m, uint32_t n, uint32_t k, uint32_t ldy,
                 uint32_t splits, uint32_t per, float* part, hipStream_t stream, bool reduce = true) {
    switch (tile) {
    case 4: launch_lds<T, 1>(w, row_bytes, xb, xscale, bias, residual, y, m, n, k, ldy, splits, per, part, stream, reduce); break;
    case 5: launch_lds<T, 2>(w, row_bytes, xb, xscale, bias, residual, y, m, n, k, ldy, splits, per, part, stream, reduce); break;
    case 0: launch_tile<T, 1, 1>(w, row_bytes, xb, xscale, bias, residual, y, m, n, k, ldy, splits, per, part, stream, reduce); break;
    case 1: launch_tile<T, 1, 2>(w, row_bytes, xb, xscale, bias, residual, y, m, n, k, ldy, splits, per, part, stream, reduce); break;
    case 2: launch_tile<T, 2, 2>(w, row_bytes, xb, xscale, bias, residual, y, m, n, k, ldy, splits, per, part, stream, reduce); break;
    case 3: launch_tile<T, 2, 4>(w, row_bytes, xb, xscale, bias, residual, y, m, n, k, ldy, splits, per, part, stream, reduce); break;
    case 6: launch_tile<T, 1, 4>(w, row_bytes, xb, xscale, bias, residual, y, m, n, k, ldy, splits, per, part, stream, reduce); break;
    default: return kInvalidArgument;
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

}  // namespace

// Tile choice: 0 = 128 x 32, 1 = 128 x 64, 2 = 256 x 64, 3 = 256 x 128,
// 6 = 128 x 128 (weight rows x X rows per block, dequantized in registers),
// 4 = 128 x 128 and 5 = 128 x 256 (dequantized once into LDS). Measured on
// the 7B prefill shapes (Q4_K, k = 3584, n = 18944): 128 x 64 (four waves per
// SIMD) is fastest up to 512 rows (M 128: 55 us against 58 for 128 x 128);
// from 1024 rows 128 x 128 in registers converts each weight half as often
// and wins despite two waves per SIMD (M 1024: 212 against 233 us, M 2048:
// 394 against 416); for long rows (the down projection, k = 18944) the
// shared-dequant 128 x 128 tile with a K split is 10-15% faster. 128 x 32 for
// a single X tile.
int gemm_default_tile(uint32_t m, uint32_t n, uint32_t k) {
    // 128 x 32 up to 64 rows of up to 8192 outputs: twice the blocks of
    // 128 x 64 (Q6_K 2048 -> 8192 at m 64: 25.1 -> 20.7 us); wider
    // matrices fill the chip either way.
    if (m <= 32 || (m <= 64 && n <= 8192)) return 0;
    // Long k (FFN down projections): the 128 x 128 register tile from 256
    // rows; it measured faster than the shared-dequant tiles at every m
    // (Q6_K 18944 -> 3584: m 256 136 -> 88 us, m 2048 546 -> 444 us).
    if (k >= 8192) return m >= 256 ? 6 : 1;
    return m >= 1024 ? 6 : 1;
}

int launch_rmsnorm_f16(const float* x, const float* gamma, float* norm, void* xh, float* xscale, size_t m, size_t k,
                       float eps, hipStream_t stream) {
    if (!x || !gamma || !norm || !xh || !xscale || m == 0 || k == 0 || k % 16 != 0 || k > 8192 || !(eps > 0.0f)) {
        return kInvalidArgument;
    }
    for (const void* p : {static_cast<const void*>(x), static_cast<const void*>(gamma), static_cast<const void*>(norm),
                          static_cast<const void*>(xh)}) {
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return kInvalidArgument;
    }
    if (m > 0x7fffffffull) return kLengthError;
    HIPLLM_LAUNCH(rmsnorm_f16_kernel, dim3(static_cast<uint32_t>(m)), dim3(256), 0, stream, x, gamma, norm,
                  static_cast<_Float16*>(xh), xscale, static_cast<uint32_t>(k), eps);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

int launch_to_f16(const float* x, size_t ldx, void* xh, float* xscale, size_t m, size_t k, hipStream_t stream) {
    if (!x || !xh || !xscale || m == 0 || k == 0 || k % 8 != 0 || ldx < k || ldx % 4 != 0) return kInvalidArgument;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(xh) % 16 != 0) return kInvalidArgument;
    if (m > 0x7fffffffull || k > 0xffffffffull) return kLengthError;
    const uint32_t chunks = static_cast<uint32_t>((k + kF16Chunk - 1) / kF16Chunk);
    HIPLLM_LAUNCH(to_f16_kernel, dim3(static_cast<uint32_t>(m), chunks), dim3(256), 0, stream, x, ldx,
                       static_cast<_Float16*>(xh), xscale, static_cast<uint32_t>(k));
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

// K splits: enough blocks for about two per CU (one for the LDS tiles, which
// hold two blocks per CU at most), each split at least two 128-k steps long
// (the X tile is double-buffered over steps). Grids of a few tiles (the
// qwen35moe projections of short prompts: 1 to 64 tiles of 2048-long rows)
// take up to eight splits where four 128-k steps per split allowed four.
uint32_t gemm_default_splits(uint32_t m, uint32_t n, uint32_t k, int tile) {
    const uint32_t bn[7] = {128, 128, 256, 256, 128, 128, 128}, bm[7] = {32, 64, 64, 128, 128, 256, 128};
    const uint64_t blocks = static_cast<uint64_t>((n + bn[tile] - 1) / bn[tile]) * ((m + bm[tile] - 1) / bm[tile]);
    const uint64_t target = tile == 4 || tile == 5 ? 256 : 512;
    const uint32_t steps = k / kStepK;
    if (blocks >= target * 3 / 4 || steps < 4) return 1;
    // Long k on the register tiles: as many splits as keep the grid within
    // 448 blocks (one round of resident blocks; each split plane also costs
    // the reduce m * n * 8 bytes of traffic).
    if (k >= 8192 && tile != 4 && tile != 5) {
        return max(1u, min(static_cast<uint32_t>(448 / blocks), steps / 2));
    }
    const uint32_t want = static_cast<uint32_t>((target + blocks - 1) / blocks);
    return max(1u, min(want, steps / 2));
}

namespace {
// The split count a launch uses: the request (0 = default), rounded so every
// split gets at least one 128-k step; *per = steps per split.
uint32_t effective_splits(uint32_t m, uint32_t n, uint32_t k, int tile, int splits, uint32_t* per) {
    const uint32_t steps = k / kStepK;
    uint32_t s = splits == 0 ? gemm_default_splits(m, n, k, tile) : static_cast<uint32_t>(splits);
    s = max(1u, min(s, steps));
    *per = (steps + s - 1) / s;
    return (steps + *per - 1) / *per;
}
}  // namespace

size_t gemm_split_bytes(size_t m, size_t n, size_t k, int tile, int splits) {
    if (m == 0 || n == 0 || k < kStepK || m > 0x7fffffffull || n > 0x7fffffffull || k > 0x7fffffffull) return 0;
    if (tile < 0) tile = gemm_default_tile(static_cast<uint32_t>(m), static_cast<uint32_t>(n), static_cast<uint32_t>(k));
    if (tile > 6 || splits < 0 || splits > 1024) return 0;
    uint32_t per;
    const uint32_t s = effective_splits(static_cast<uint32_t>(m), static_cast<uint32_t>(n), static_cast<uint32_t>(k),
                                        tile, splits, &per);
    return s > 1 ? static_cast<size_t>(s) * m * n * sizeof(float) : 0;
}

int launch_gemm_mfma(uint32_t type, const void* w, size_t row_bytes, const void* xb, const float* xscale,
                     const float* bias, const float* residual, float* y, size_t m, size_t n, size_t k, int tile,
                     int splits, hipStream_t stream, size_t ldy, void* split_ws, size_t split_ws_bytes) {
    if (ldy == 0) ldy = n;
    if (!w || !xb || !xscale || !y || m == 0 || n == 0 || k == 0 || ldy < n || ldy > 0x7fffffffull) return kInvalidArgument;
    if (k % kStepK != 0) return kInvalidArgument;
    if (m > 0x7fffffffull || n > 0x7fffffffull || k > 0x7fffffffull) return kLengthError;
    if (((n + 127) / 128) * ((m + 31) / 32) > 0x7fffffffull) return kLengthError;  // one grid row of tiles
    if (type != kF32 && type != kF16 && type != kQ5_0 && type != kQ8_0 && type != kQ4_K && type != kQ6_K) {
        return kInvalidArgument;
    }
    if (row_bytes < k / block_elems(type) * block_bytes(type)) return kInvalidArgument;
    if (reinterpret_cast<uintptr_t>(w) % 2 != 0 || row_bytes % 2 != 0) return kInvalidArgument;
    if ((type == kQ4_K || type == kF32 || type == kF16) &&
        (reinterpret_cast<uintptr_t>(w) % 4 != 0 || row_bytes % 4 != 0)) {
        return kInvalidArgument;
    }
    if (reinterpret_cast<uintptr_t>(xb) % 16 != 0) return kInvalidArgument;
    if (tile < 0) tile = gemm_default_tile(static_cast<uint32_t>(m), static_cast<uint32_t>(n), static_cast<uint32_t>(k));
    if (tile > 6) return kInvalidArgument;
    const uint32_t M = static_cast<uint32_t>(m), N = static_cast<uint32_t>(n), K = static_cast<uint32_t>(k);
    if (splits < 0 || splits > 1024) return kInvalidArgument;
    uint32_t per;
    uint32_t S = effective_splits(M, N, K, tile, splits, &per);
    const size_t need = S > 1 ? static_cast<size_t>(S) * m * n * sizeof(float) : 0;
    if (need > split_ws_bytes || (need && !split_ws)) {
        // An explicit split needs its partial-sum planes; the default split
        // falls back to one pass over k.
        if (splits != 0) return kInvalidArgument;
        S = 1;
        per = K / kStepK;
    }
    if (S > 1 && reinterpret_cast<uintptr_t>(split_ws) % 16 != 0) return kInvalidArgument;
    float* part = static_cast<float*>(split_ws);
    const auto* x = static_cast<const _Float16*>(xb);
    const uint32_t LD = static_cast<uint32_t>(ldy);
    switch (type) {
    case kQ4_K: return launch_typed<kQ4_K>(tile, w, row_bytes, x, xscale, bias, residual, y, M, N, K, LD, S, per, part, stream);
    case kQ6_K: return launch_typed<kQ6_K>(tile, w, row_bytes, x, xscale, bias, residual, y, M, N, K, LD, S, per, part, stream);
    case kQ8_0: return launch_typed<kQ8_0>(tile, w, row_bytes, x, xscale, bias, residual, y, M, N, K, LD, S, per, part, stream);
    case kQ5_0: return launch_typed<kQ5_0>(tile, w, row_bytes, x, xscale, bias, residual, y, M, N, K, LD, S, per, part, stream);
    case kF32: return launch_typed<kF32>(tile, w, row_bytes, x, xscale, bias, residual, y, M, N, K, LD, S, per, part, stream);
    case kF16: return launch_typed<kF16>(tile, w, row_bytes, x, xscale, bias, residual, y, M, N, K, LD, S, per, part, stream);
    default: return kInvalidArgument;
    }
}

// The FFN gate and up matmuls of a prompt and their SwiGLU: both products
// keep their K-split partial planes (or, unsplit, one plane each) in the
// workspace, and one launch adds each product's planes in split order and
// applies the sign-branched SwiGLU (swiglu_kernel's expression), saving the
// two split reductions' and the SwiGLU launch's passes over the rows.
__global__ __launch_bounds__(256) void gemm_split_swiglu_kernel(const float* __restrict__ pg,
                                                                const float* __restrict__ pu, uint32_t splits,
                                                                float* __restrict__ y, uint32_t m, uint32_t n,
                                                                uint32_t ldy) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t plane = static_cast<size_t>(m) * n;
    if (i >= plane) return;
    float g = pg[i], u = pu[i];
    for (uint32_t z = 1; z < splits; ++z) {
        g += pg[z * plane + i];
        u += pu[z * plane + i];
    }
    const float sig = g >= 0.0f ? 1.0f / (1.0f + expf(-g)) : expf(g) / (1.0f + expf(g));
    y[(i / n) * ldy + i % n] = g * sig * u;
}

// gemm_split_swiglu_kernel's row followed by to_f16_kernel's conversion of
// it, in one launch: block r (1024 threads) forms the n SwiGLU values of row
// r from the planes as there (8 per thread and group, at most 32 per
// thread, kept in registers), reduces the row's largest magnitude, and
// writes the fp16 row and its scale as to_f16_kernel does: the same bits as
// the two launches, without the FP32 row in memory. n % 8 == 0,
// n <= kSwigluF16Max.
constexpr uint32_t kSwigluF16Max = 32768;
__global__ __launch_bounds__(1024) void gemm_split_swiglu_f16_kernel(const float* __restrict__ pg,
                                                                     const float* __restrict__ pu, uint32_t splits,
                                                                     _Float16* __restrict__ yh,
                                                                     float* __restrict__ yscale, uint32_t m,
                                                                     uint32_t n) {
    constexpr uint32_t kGroups = kSwigluF16Max / 8 / 1024;
    const uint32_t r = blockIdx.x, tid = threadIdx.x;
    const size_t plane = static_cast<size_t>(m) * n;
    const size_t row0 = static_cast<size_t>(r) * n;
    float v[kGroups][8];
    float mx = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < kGroups; ++j) {
        const uint32_t c = 8 * (tid + 1024 * j);
        if (c < n) {
#pragma unroll
            for (uint32_t h = 0; h < 2; ++h) {
                const size_t i = row0 + c + 4 * h;
                float4 g = *reinterpret_cast<const float4*>(pg + i), u = *reinterpret_cast<const float4*>(pu + i);
                for (uint32_t z = 1; z < splits; ++z) {
                    const float4 gz = *reinterpret_cast<const float4*>(pg + z * plane + i);
                    const float4 uz = *reinterpret_cast<const float4*>(pu + z * plane + i);
                    g.x += gz.x; g.y += gz.y; g.z += gz.z; g.w += gz.w;
                    u.x += uz.x; u.y += uz.y; u.z += uz.z; u.w += uz.w;
                }
                const float gg[4] = {g.x, g.y, g.z, g.w}, uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (uint32_t q = 0; q < 4; ++q) {
                    const float a = gg[q];
                    const float sig = a >= 0.0f ? 1.0f / (1.0f + expf(-a)) : expf(a) / (1.0f + expf(a));
                    const float y = a * sig * uu[q];
                    v[j][4 * h + q] = y;
                    mx = fmaxf(mx, fabsf(y));
                }
            }
        }
    }
    __shared__ float red[16];
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
    for (uint32_t w = 1; w < 16; ++w) mx = fmaxf(mx, red[w]);
    int e = 0;
    if (mx > 0.0f && mx <= 3.402823466e38f) {
        frexpf(mx, &e);
        e = max(-126, min(127, e - 14));
    }
    const float down = ldexpf(1.0f, -e);
    if (tid == 0) yscale[r] = ldexpf(1.0f, e);
#pragma unroll
    for (uint32_t j = 0; j < kGroups; ++j) {
        const uint32_t c = 8 * (tid + 1024 * j);
        if (c < n) {
            const u32x4 o = {pack_h2(v[j][0] * down, v[j][1] * down), pack_h2(v[j][2] * down, v[j][3] * down),
                             pack_h2(v[j][4] * down, v[j][5] * down), pack_h2(v[j][6] * down, v[j][7] * down)};
            *reinterpret_cast<u32x4*>(yh + row0 + c) = o;
        }
    }
}

size_t gemm_swiglu_bytes(size_t m, size_t n, size_t k) {
    if (m == 0 || n == 0 || k < kStepK || m > 0x7fffffffull || n > 0x7fffffffull || k > 0x7fffffffull) return 0;
    uint32_t per;
    const uint32_t M = static_cast<uint32_t>(m), N = static_cast<uint32_t>(n), K = static_cast<uint32_t>(k);
    const uint32_t s = effective_splits(M, N, K, gemm_default_tile(M, N, K), 0, &per);
    return 2 * static_cast<size_t>(s) * m * n * sizeof(float);
}

int launch_gemm_mfma_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const void* xb,
                            const float* xscale, float* y, size_t m, size_t n, size_t k, size_t ldy, void* ws,
                            size_t ws_bytes, hipStream_t stream, void* yh, float* yscale) {
    if (ldy == 0) ldy = n;
    const bool f16 = yh != nullptr;
    if (f16 && (!yscale || n % 8 != 0 || n > kSwigluF16Max || reinterpret_cast<uintptr_t>(yh) % 16 != 0)) {
        return kInvalidArgument;
    }
    if (!wg || !wu || !xb || !xscale || (!y && !f16) || !ws || m == 0 || n == 0 || k == 0 || ldy < n || ldy > 0x7fffffffull ||
        k % kStepK != 0) {
        return kInvalidArgument;
    }
    if (m > 0x7fffffffull || n > 0x7fffffffull || k > 0x7fffffffull) return kLengthError;
    if (type != kQ5_0 && type != kQ8_0 && type != kQ4_K && type != kQ6_K) return kInvalidArgument;
    if (row_bytes < k / block_elems(type) * block_bytes(type) || row_bytes % 2 != 0) return kInvalidArgument;
    for (const void* p : {wg, wu}) {
        if (reinterpret_cast<uintptr_t>(p) % (type == kQ4_K ? 4 : 2) != 0) return kInvalidArgument;
    }
    if (type == kQ4_K && row_bytes % 4 != 0) return kInvalidArgument;
    if (reinterpret_cast<uintptr_t>(xb) % 16 != 0 || reinterpret_cast<uintptr_t>(ws) % 16 != 0) return kInvalidArgument;
    const size_t need = gemm_swiglu_bytes(m, n, k);
    if (need == 0 || need > ws_bytes) return kInvalidArgument;
    const uint32_t M = static_cast<uint32_t>(m), N = static_cast<uint32_t>(n), K = static_cast<uint32_t>(k);
    const int tile = gemm_default_tile(M, N, K);
    uint32_t per;
    const uint32_t S = effective_splits(M, N, K, tile, 0, &per);
    float* pg = static_cast<float*>(ws);
    float* pu = pg + static_cast<size_t>(S) * m * n;
    const auto* x = static_cast<const _Float16*>(xb);
    // Unsplit, each product writes its one plane as y with ldy = n; split, its planes (no reduce).
    int rc = kOk;
    for (int j = 0; j < 2 && rc == kOk; ++j) {
        const void* w = j == 0 ? wg : wu;
        float* p = j == 0 ? pg : pu;
        switch (type) {
        case kQ4_K: rc = launch_typed<kQ4_K>(tile, w, row_bytes, x, xscale, nullptr, nullptr, p, M, N, K, N, S, per, p, stream, false); break;
        case kQ6_K: rc = launch_typed<kQ6_K>(tile, w, row_bytes, x, xscale, nullptr, nullptr, p, M, N, K, N, S, per, p, stream, false); break;
        case kQ8_0: rc = launch_typed<kQ8_0>(tile, w, row_bytes, x, xscale, nullptr, nullptr, p, M, N, K, N, S, per, p, stream, false); break;
        default: rc = launch_typed<kQ5_0>(tile, w, row_bytes, x, xscale, nullptr, nullptr, p, M, N, K, N, S, per, p, stream, false); break;
        }
    }
    if (rc != kOk) return rc;
    if (f16) {
        HIPLLM_LAUNCH(gemm_split_swiglu_f16_kernel, dim3(M), dim3(1024), 0, stream, pg, pu, S,
                      static_cast<_Float16*>(yh), yscale, M, N);
        return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
    }
    const size_t total = static_cast<size_t>(m) * n;
    HIPLLM_LAUNCH(gemm_split_swiglu_kernel, dim3(static_cast<uint32_t>((total + 255) / 256)), dim3(256), 0, stream, pg,
                  pu, S, y, M, N, static_cast<uint32_t>(ldy));
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

int launch_gemm_gather(uint32_t type, const void* w, size_t row_bytes, const void* xb, const float* xscale, float* y,
                       size_t n, size_t k, size_t ldy, const int32_t* order, const int32_t* groups,
                       const uint32_t* ngroups, size_t max_groups, size_t expert_stride, size_t routes, int x_routed,
                       hipStream_t stream) {
    if (!w || !xb || !xscale || !y || !order || !groups || !ngroups || n == 0 || k == 0 || max_groups == 0 || routes == 0 ||
        ldy < n) {
        return kInvalidArgument;
    }
    if (k % kStepK != 0) return kInvalidArgument;
    if (n > 0x7fffffffull || k > 0x7fffffffull || ldy > 0x7fffffffull || max_groups > 65535 ||
        routes > 0xffffffffull) {
        return kLengthError;
    }
    if (type != kF32 && type != kF16 && type != kQ5_0 && type != kQ8_0 && type != kQ4_K && type != kQ6_K) {
        return kInvalidArgument;
    }
    if (row_bytes < k / block_elems(type) * block_bytes(type) || expert_stride < n * row_bytes) {
        return kInvalidArgument;
    }
    if (reinterpret_cast<uintptr_t>(w) % 2 != 0 || row_bytes % 2 != 0 || expert_stride % 2 != 0) {
        return kInvalidArgument;
    }
    if ((type == kQ4_K || type == kF32 || type == kF16) &&
        (reinterpret_cast<uintptr_t>(w) % 4 != 0 || row_bytes % 4 != 0 || expert_stride % 4 != 0)) {
        return kInvalidArgument;
    }
    if (reinterpret_cast<uintptr_t>(xb) % 16 != 0) return kInvalidArgument;
    Gather g;
    g.order = order;
    g.groups = groups;
    g.ngroups = ngroups;
    g.expert_stride = expert_stride;
    g.routes = static_cast<uint32_t>(routes);
    g.x_routed = x_routed ? 1u : 0u;
    const auto* x = static_cast<const _Float16*>(xb);
    const uint32_t N = static_cast<uint32_t>(n), K = static_cast<uint32_t>(k), L = static_cast<uint32_t>(ldy);
    const uint32_t G = static_cast<uint32_t>(max_groups);
    switch (type) {
    case kQ4_K: launch_gather<kQ4_K>(w, row_bytes, x, xscale, y, N, K, L, G, g, stream); break;
    case kQ6_K: launch_gather<kQ6_K>(w, row_bytes, x, xscale, y, N, K, L, G, g, stream); break;
    case kQ8_0: launch_gather<kQ8_0>(w, row_bytes, x, xscale, y, N, K, L, G, g, stream); break;
    case kQ5_0: launch_gather<kQ5_0>(w, row_bytes, x, xscale, y, N, K, L, G, g, stream); break;
    case kF32: launch_gather<kF32>(w, row_bytes, x, xscale, y, N, K, L, G, g, stream); break;
    default: launch_gather<kF16>(w, row_bytes, x, xscale, y, N, K, L, G, g, stream); break;
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

}  // namespace hipllm
