// Decode GEMV over native GGUF block-quantized weights: y[N] = W[N,K] x[K].
//
// Replaces the reference's one-thread-per-row GEVMs (metal_llm.metal:708-781,
// dot_q*_f32 319-553; host encode_vector_product metal_llm.mm:1891-1999) with
// a wave-cooperative design for CDNA4:
//
// * An "octet" of 8 lanes owns one unit of a row (a 256-value super-block for
//   Q4_K / Q6_K / F32 / F16, two 32-value blocks for Q8_0 / Q5_0). Every lane
//   issues 128-bit loads of its slice of the unit, so eight lanes read one
//   contiguous super-block.
// * Each octet computes R rows at once: a lane loads its activation slice of a
//   unit once and multiplies it into the same slice of R rows, so activation
//   traffic through the vector L1 is 1/R of the weight-side element count.
//   This is what keeps the kernel on the HBM roofline rather than the L1 one.
// * OPR octets share a row group and split its units round-robin (K split
//   inside the wave); a wave holds 8 / OPR row groups, a block 4 waves.
//   (R, OPR) is chosen per shape so every shape launches >= ~1000 waves.
// * Values are dequantized in registers to FP32 and accumulated in FP32. The
//   constant part of each affine block format (Q4_K's -dmin*m, Q6_K's -32,
//   Q8_0's -128 after the sign flip, Q5_0's -16) is applied once per 16-group
//   via per-16 sums of x (xs16) that the activation's producer writes.
//   Nibbles and bytes turn into floats with v_cvt_f32_ubyte{0..3}.
// * Q4_K's 16-byte super-block header is fetched as one dword per lane and
//   spread across each quad of lanes with DPP broadcasts.
// * Partials reduce with lane shuffles in a fixed order (deterministic); the
//   epilogue adds bias and residual, or applies SwiGLU for the fused gate/up
//   form and writes the per-16 sums the down projection consumes.
//
// Weight rows may be only 2-byte aligned (Q6_K / Q8_0 / Q5_0 block sizes are
// 210 / 34 / 22 bytes); such loads read the enclosing aligned dwords and
// realign with v_alignbyte. Device weight buffers carry 256 bytes of tail
// padding so those reads stay in bounds.
#include "common.h"
#include "launch.h"

namespace hipllm {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

namespace {

__device__ __forceinline__ uint4 ld128_a4(const uint8_t* p) {
    const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes from a 2-byte-aligned address.
__device__ __forceinline__ uint4 ld128_a2(const uint8_t* p) {
    const uint32_t s = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint8_t* base = p - s;  // pointer arithmetic keeps the global address space
    const uint4 v = ld128_a4(base);
    const uint32_t e = *reinterpret_cast<const uint32_t*>(base + 16);
    return make_uint4(__builtin_amdgcn_alignbyte(v.y, v.x, s), __builtin_amdgcn_alignbyte(v.z, v.y, s),
                      __builtin_amdgcn_alignbyte(v.w, v.z, s), __builtin_amdgcn_alignbyte(e, v.w, s));
}

// Hides a value's known bits from the instruction combiner so byte extracts
// of it select v_cvt_f32_ubyte{1,2,3} instead of shift + bit-field extract.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}

__device__ __forceinline__ float dot4_u8(uint32_t q, float4 xv, float acc) {
    acc = fmaf(xv.x, ubyte0(q), acc);
    acc = fmaf(xv.y, ubyte1(q), acc);
    acc = fmaf(xv.z, ubyte2(q), acc);
    acc = fmaf(xv.w, ubyte3(q), acc);
    return acc;
}

__device__ __forceinline__ float4 ldx4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// Value of lane I of this lane's quad (DPP quad_perm broadcast).
template <int I>
__device__ __forceinline__ uint32_t quad_lane(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(v), I * 0x55, 0xf, 0xf, false));
}

template <uint32_t T>
struct Unit;

// Q4_K: 144-byte super-block {d, dmin, scales[12], qs[128]}. Lane c of the
// octet takes qs bytes [16c, 16c+16): group j = c/2, l0 = 16 (c & 1); its low
// nibbles are elements 64j+l0.. of sub-block 2j, its high nibbles elements
// 64j+32+l0.. of sub-block 2j+1 (model.cpp:616-644). High nibbles are kept in
// place (16 q) and the 1/16 folds into the sub-block scale.
template <>
struct Unit<kQ4_K> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 144;
    struct X {
        float4 a[4], b[4];
        float sl, sh;
    };
    __device__ static __forceinline__ X load_x(const float* x, const float* xs16, uint32_t c) {
        const uint32_t j = c >> 1;
        const uint32_t l0 = (c & 1) * 16;
        const float* xl = x + 64 * j + l0;
        X v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v.a[i] = ldx4(xl + 4 * i);
            v.b[i] = ldx4(xl + 32 + 4 * i);
        }
        v.sl = xs16[(64 * j + l0) >> 4];
        v.sh = xs16[(64 * j + 32 + l0) >> 4];
        return v;
    }
    struct W {
        uint32_t head;  // header dword (c & 3)
        uint4 q;
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        W w;
        w.head = *reinterpret_cast<const uint32_t*>(u + 4 * (c & 3));
        w.q = ld128_a4(u + 16 + 16 * c);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t c, const X& xv) {
        const uint32_t h0 = quad_lane<0>(w.head), h1 = quad_lane<1>(w.head);
        const uint32_t h2 = quad_lane<2>(w.head), h3 = quad_lane<3>(w.head);
        const uint32_t j = c >> 1;
        // 6-bit scale/min pairs of all eight sub-blocks as packed bytes
        // (get_scale_min_k4, model.cpp:524-537), then this lane's two.
        uint32_t S, M;
        if (j < 2) {
            S = h1 & 0x3f3f3f3fu;
            M = h2 & 0x3f3f3f3fu;
        } else {
            S = (h3 & 0x0f0f0f0fu) | ((h1 >> 2) & 0x30303030u);
            M = ((h3 >> 4) & 0x0f0f0f0fu) | ((h2 >> 2) & 0x30303030u);
        }
        const uint32_t sh16 = (j & 1) * 16;
        S >>= sh16;
        M >>= sh16;
        const float d = half_lo(h0);
        const float dmin = half_hi(h0);
        float s0 = 0.0f, s1 = 0.0f;
        const uint32_t Q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s0 = dot4_u8(opaque(Q[i] & 0x0f0f0f0fu), xv.a[i], s0);
            s1 = dot4_u8(opaque(Q[i] & 0xf0f0f0f0u), xv.b[i], s1);
        }
        const float r0 = d * ubyte0(S) * s0 - dmin * ubyte0(M) * xv.sl;
        const float r1 = d * (ubyte1(S) * 0.0625f) * s1 - dmin * ubyte1(M) * xv.sh;
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
    struct X {
        float4 a[4], b[4];
        float sa, sb;
    };
    __device__ static __forceinline__ X load_x(const float* x, const float* xs16, uint32_t c) {
        const uint32_t n = c >> 2, m = (c >> 1) & 1, hh = c & 1;
        const uint32_t e0 = 128 * n + 32 * m + 16 * hh;
        X v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v.a[i] = ldx4(x + e0 + 4 * i);
            v.b[i] = ldx4(x + e0 + 64 + 4 * i);
        }
        v.sa = 32.0f * xs16[e0 >> 4];
        v.sb = 32.0f * xs16[(e0 + 64) >> 4];
        return v;
    }
    struct W {
        uint4 ql, qh;
        uint32_t sc;  // scale bytes sA (bits 0..7) and sB (8..15)
        uint32_t d;
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        const uint32_t n = c >> 2, m = (c >> 1) & 1, hh = c & 1;
        W w;
        w.ql = ld128_a2(u + 64 * n + 32 * m + 16 * hh);
        w.qh = ld128_a2(u + 128 + 32 * n + 16 * hh);
        // scales[16] and d: bytes 192..209.
        const uint32_t ts = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(u + 192) & 3u);
        const uint8_t* tb = u + 192 - ts;
        const uint4 t = ld128_a4(tb);
        const uint32_t t4 = *reinterpret_cast<const uint32_t*>(tb + 16);
        const uint32_t sc0_3 = __builtin_amdgcn_alignbyte(t.y, t.x, ts);
        const uint32_t sc4_7 = __builtin_amdgcn_alignbyte(t.z, t.y, ts);
        const uint32_t sc8_11 = __builtin_amdgcn_alignbyte(t.w, t.z, ts);
        const uint32_t sc12_15 = __builtin_amdgcn_alignbyte(t4, t.w, ts);
        // Scale bytes used: index 8n + hh + 2m (low nibbles) and +4 (high).
        const uint32_t wlo = n ? sc8_11 : sc0_3;
        const uint32_t whi = n ? sc12_15 : sc4_7;
        const uint32_t sel = 8 * (hh + 2 * m);
        w.sc = ((wlo >> sel) & 0xffu) | (((whi >> sel) & 0xffu) << 8);
        w.d = __builtin_amdgcn_alignbyte(t4, t4, ts) & 0xffffu;  // bytes 16..17 of the tail
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t c, const X& xv) {
        const uint32_t m = (c >> 1) & 1;
        const uint32_t shl = 4 - 2 * m;  // qh bits (2m, 2m+1) -> bits 4, 5
        const uint32_t shr = 2 * m;      // qh bits (2m+4, 2m+5) -> bits 4, 5
        float s0 = 0.0f, s1 = 0.0f;
        const uint32_t L[4] = {w.ql.x, w.ql.y, w.ql.z, w.ql.w};
        const uint32_t H[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (L[i] & 0x0f0f0f0fu) | ((H[i] << shl) & 0x30303030u);
            const uint32_t hi = ((L[i] >> 4) & 0x0f0f0f0fu) | ((H[i] >> shr) & 0x30303030u);
            s0 = dot4_u8(opaque(lo), xv.a[i], s0);
            s1 = dot4_u8(opaque(hi), xv.b[i], s1);
        }
        const float d = half_lo(w.d);
        const float sA = static_cast<float>(static_cast<int8_t>(w.sc & 0xffu));
        const float sB = static_cast<float>(static_cast<int8_t>((w.sc >> 8) & 0xffu));
        // value = d * sc * (q - 32)
        return d * sA * (s0 - xv.sa) + d * sB * (s1 - xv.sb);
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
    struct X {
        float4 a, b;
        float s;
    };
    __device__ static __forceinline__ X load_x(const float* x, const float* xs16, uint32_t c) {
        const uint32_t b = c >> 2, p = c & 3;
        const uint32_t e0 = 32 * b + 8 * p;
        X v;
        v.a = ldx4(x + e0);
        v.b = ldx4(x + e0 + 4);
        v.s = (p & 1) == 0 ? 128.0f * xs16[e0 >> 4] : 0.0f;
        return v;
    }
    struct W {
        uint2 q;
        uint32_t d;
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        const uint32_t b = c >> 2, p = c & 3;
        const uint8_t* blk = u + 34 * b;
        W w;
        w.d = load_u16_a2(blk);
        w.q = load_u64_a2(blk + 2 + 8 * p);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t, const X& xv) {
        float s = 0.0f;
        s = dot4_u8(opaque(w.q.x ^ 0x80808080u), xv.a, s);
        s = dot4_u8(opaque(w.q.y ^ 0x80808080u), xv.b, s);
        return half_lo(w.d) * (s - xv.s);
    }
};

// Q5_0: two 22-byte blocks {d, qh[4], qs[16]} per unit. Lane c = (b, p)
// takes qs bytes [4p, 4p+4) of block b: low nibbles are elements 32b+4p+i,
// high nibbles 32b+16+4p+i; the fifth bits come from qh (model.cpp:581-601).
template <>
struct Unit<kQ5_0> {
    static constexpr uint32_t elems = 64;
    static constexpr uint32_t bytes = 44;
    struct X {
        float4 a, b;
        float s;
    };
    __device__ static __forceinline__ X load_x(const float* x, const float* xs16, uint32_t c) {
        const uint32_t b = c >> 2, p = c & 3;
        const uint32_t e0 = 32 * b + 4 * p;
        X v;
        v.a = ldx4(x + e0);
        v.b = ldx4(x + e0 + 16);
        v.s = p == 0 ? 16.0f * (xs16[(32 * b) >> 4] + xs16[(32 * b + 16) >> 4]) : 0.0f;
        return v;
    }
    struct W {
        uint32_t d, qh, qs;
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        const uint32_t b = c >> 2, p = c & 3;
        const uint8_t* blk = u + 22 * b;
        W w;
        w.d = load_u16_a2(blk);
        w.qh = load_u32_a2(blk + 2);
        w.qs = load_u32_a2(blk + 6 + 4 * p);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t c, const X& xv) {
        const uint32_t p = c & 3;
        const uint32_t hlo = (w.qh >> (4 * p)) & 0xfu;
        const uint32_t hhi = (w.qh >> (16 + 4 * p)) & 0xfu;
        const uint32_t lo = (w.qs & 0x0f0f0f0fu) | (((hlo * 0x00204081u) & 0x01010101u) << 4);
        const uint32_t hi = ((w.qs >> 4) & 0x0f0f0f0fu) | (((hhi * 0x00204081u) & 0x01010101u) << 4);
        float s = 0.0f;
        s = dot4_u8(opaque(lo), xv.a, s);
        s = dot4_u8(opaque(hi), xv.b, s);
        return half_lo(w.d) * (s - xv.s);
    }
};

// F32: 256 values (1024 bytes) per unit; lane c takes values [32c, 32c+32).
template <>
struct Unit<kF32> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 1024;
    struct X {
        float4 a[8];
    };
    __device__ static __forceinline__ X load_x(const float* x, const float*, uint32_t c) {
        X v;
#pragma unroll
        for (int i = 0; i < 8; ++i) v.a[i] = ldx4(x + 32 * c + 4 * i);
        return v;
    }
    struct W {
        float4 w[8];
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        W w;
        const float* p = reinterpret_cast<const float*>(u) + 32 * c;
#pragma unroll
        for (int i = 0; i < 8; ++i) w.w[i] = ldx4(p + 4 * i);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t, const X& xv) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s = fmaf(w.w[i].x, xv.a[i].x, s);
            s = fmaf(w.w[i].y, xv.a[i].y, s);
            s = fmaf(w.w[i].z, xv.a[i].z, s);
            s = fmaf(w.w[i].w, xv.a[i].w, s);
        }
        return s;
    }
};

// F16: 256 values (512 bytes) per unit; lane c takes values [32c, 32c+32).
template <>
struct Unit<kF16> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 512;
    struct X {
        float4 a[8];
    };
    __device__ static __forceinline__ X load_x(const float* x, const float*, uint32_t c) {
        X v;
#pragma unroll
        for (int i = 0; i < 8; ++i) v.a[i] = ldx4(x + 32 * c + 4 * i);
        return v;
    }
    struct W {
        uint4 h[4];
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        W w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w.h[i] = ld128_a4(u + 64 * c + 16 * i);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t, const X& xv) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s = fmaf(half_lo(w.h[i].x), xv.a[2 * i].x, s);
            s = fmaf(half_hi(w.h[i].x), xv.a[2 * i].y, s);
            s = fmaf(half_lo(w.h[i].y), xv.a[2 * i].z, s);
            s = fmaf(half_hi(w.h[i].y), xv.a[2 * i].w, s);
            s = fmaf(half_lo(w.h[i].z), xv.a[2 * i + 1].x, s);
            s = fmaf(half_hi(w.h[i].z), xv.a[2 * i + 1].y, s);
            s = fmaf(half_lo(w.h[i].w), xv.a[2 * i + 1].z, s);
            s = fmaf(half_hi(w.h[i].w), xv.a[2 * i + 1].w, s);
        }
        return s;
    }
};

// Sign-branched SiLU gate as in the reference SwiGLU (cpu_llm.cpp:188-202).
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float sig = g >= 0.0f ? 1.0f / (1.0f + expf(-g)) : expf(g) / (1.0f + expf(g));
    return g * sig * u;
}

// Several GEMVs in one launch: blockIdx.y is an output row-vector index j.
// With ids (expert routing, moe_llm.mm:2692-2760; metal_expert_gemm_q*_f32
// metal_llm.metal:1476-1521) the weights of vector j are those of expert
// ids[j] (clamped to experts - 1), at byte offset ids[j] * expert_stride; the
// input is row j (x_routed) or row j / routes of x. Without ids every vector
// uses the same weights (a batch of rows through one matrix).
struct Batch {
    const int32_t* ids = nullptr;
    uint32_t experts = 1;
    uint32_t routes = 1;
    size_t expert_stride = 0;
    uint32_t x_routed = 0;
    uint32_t ldx = 0;  // floats between input rows (multiple of 16)
    uint32_t ldy = 0;  // floats between output rows
};

// R rows per octet, OPR octets per row group (K split), 8 / OPR row groups
// per wave, 4 waves per block: rows per block = 32 R / OPR.
// MODE 0: y = W x (+ bias) (+ residual).
// MODE 1: y = silu(W x) * (W2 x); each octet carries R rows of W and the same
//         R rows of W2. ys16 (optional) receives per-16 sums of y.
template <uint32_t T, int R, int OPR, int MODE>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                                                   size_t row_bytes, const float* __restrict__ x,
                                                   const float* __restrict__ xs16, const float* __restrict__ bias,
                                                   const float* __restrict__ residual, float* __restrict__ y,
                                                   float* __restrict__ ys16, uint32_t n, uint32_t units,
                                                   const Batch batch) {
    using U = Unit<T>;
    {
        // Vector j of the batch: shift weights, input, output and residual.
        const uint32_t j = blockIdx.y;
        const uint32_t xrow = batch.x_routed ? j : j / batch.routes;
        if (batch.ids) {
            const uint32_t e = min(static_cast<uint32_t>(batch.ids[j]), batch.experts - 1);
            w += static_cast<size_t>(e) * batch.expert_stride;
            if (MODE == 1) w2 += static_cast<size_t>(e) * batch.expert_stride;
        }
        x += static_cast<size_t>(xrow) * batch.ldx;
        xs16 += static_cast<size_t>(xrow) * (batch.ldx / 16);
        y += static_cast<size_t>(j) * batch.ldy;
        if (residual) residual += static_cast<size_t>(j) * batch.ldy;
        if (ys16) ys16 += static_cast<size_t>(j) * (batch.ldy / 16);
    }
    constexpr int GPW = 8 / OPR;
    constexpr int RPB = 4 * GPW * R;
    constexpr int NR = MODE == 1 ? 2 * R : R;
    static_assert(OPR == 1 || OPR == 2 || OPR == 4 || OPR == 8, "OPR must divide 8");
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t o = lane >> 3, c = lane & 7;
    const uint32_t rg = o / OPR, slot = o % OPR;
    const uint32_t lrow0 = (wave * GPW + rg) * R;  // first row of this octet within the block
    const uint32_t row0 = blockIdx.x * RPB + lrow0;

    const uint8_t* wr[NR];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const uint32_t r = min(row0 + i, n - 1);  // rows past n are computed, never stored
        wr[i] = w + static_cast<size_t>(r) * row_bytes;
        if (MODE == 1) wr[R + i] = w2 + static_cast<size_t>(r) * row_bytes;
    }
    float acc[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) acc[i] = 0.0f;

#pragma unroll 2
    for (uint32_t u = slot; u < units; u += OPR) {
        typename U::W wv[NR];
#pragma unroll
        for (int i = 0; i < NR; ++i) wv[i] = U::load_w(wr[i] + static_cast<size_t>(u) * U::bytes, c);
        const typename U::X xv = U::load_x(x + u * U::elems, xs16 + u * (U::elems / 16), c);
#pragma unroll
        for (int i = 0; i < NR; ++i) acc[i] += U::dot(wv[i], c, xv);
    }

    // Reduce the 8 lanes of the octet, then the OPR octets of the row group.
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        float v = acc[i];
        v += __shfl_xor(v, 1);
        v += __shfl_xor(v, 2);
        v += __shfl_xor(v, 4);
#pragma unroll
        for (int s = 8; s < 8 * OPR; s <<= 1) v += __shfl_xor(v, s);
        acc[i] = v;
    }
    const bool writer = c == 0 && slot == 0;
    if (MODE == 0) {
        if (writer) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const uint32_t r = row0 + i;
                if (r < n) {
                    float s = acc[i];
                    if (bias) s += bias[r];
                    if (residual) s += residual[r];
                    y[r] = s;
                }
            }
        }
    } else {
        __shared__ float outs[RPB];
        if (writer) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const uint32_t r = row0 + i;
                const float v = r < n ? silu_mul(acc[i], acc[R + i]) : 0.0f;
                outs[lrow0 + i] = v;
                if (r < n) y[r] = v;
            }
        }
        if (ys16) {
            __syncthreads();
            if (tid < static_cast<uint32_t>(RPB / 16)) {
                const uint32_t g0 = blockIdx.x * RPB + 16 * tid;
                if (g0 < n) {
                    float t = 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; ++i) t += outs[16 * tid + i];
                    ys16[g0 / 16] = t;
                }
            }
        }
    }
}

// ------------------------------------------------------------ K-sliced form
// For rows of >= 12 super-blocks (the large decode GEMVs): every wave owns a
// fixed K slice of 16 super-blocks, four lanes per super-block, and keeps the
// activation values of its slice in registers for the whole launch. A block
// holds `wpr` such waves per row (the K slices) times `teams` row teams and
// streams its row range R rows at a time: per row a lane loads 32 bytes of
// quants plus one header dword and does 64 multiply-adds, so activations are
// read once per wave instead of once per row. Each wave reduces its R partial
// sums across its 64 lanes; the per-slice partials meet in LDS and one
// thread per row adds them in slice order (deterministic), then applies the
// bias / residual or SwiGLU epilogue.
template <uint32_t T>
struct Slice;

// Q4_K: lane q (0..3) of a super-block takes qs bytes [32q, 32q + 32): low
// nibbles are elements 64q + [0, 32) (sub-block 2q), high nibbles
// 64q + 32 + [0, 32) (sub-block 2q + 1) (model.cpp:616-644).
template <>
struct Slice<kQ4_K> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 144;
    struct X {
        float4 lo[8], hi[8];
        float sl, sh;
    };
    __device__ static __forceinline__ X load_x(const float* x, const float* xs16, uint32_t q) {
        X v;
        const float* xl = x + 64 * q;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v.lo[i] = ldx4(xl + 4 * i);
            v.hi[i] = ldx4(xl + 32 + 4 * i);
        }
        v.sl = xs16[4 * q] + xs16[4 * q + 1];
        v.sh = xs16[4 * q + 2] + xs16[4 * q + 3];
        return v;
    }
    struct W {
        uint32_t head;
        uint4 q0, q1;
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t q) {
        W w;
        w.head = *reinterpret_cast<const uint32_t*>(u + 4 * q);
        w.q0 = ld128_a4(u + 16 + 32 * q);
        w.q1 = ld128_a4(u + 32 + 32 * q);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t q, const X& xv) {
        const uint32_t h0 = quad_lane<0>(w.head), h1 = quad_lane<1>(w.head);
        const uint32_t h2 = quad_lane<2>(w.head), h3 = quad_lane<3>(w.head);
        uint32_t S, M;
        if (q < 2) {
            S = h1 & 0x3f3f3f3fu;
            M = h2 & 0x3f3f3f3fu;
        } else {
            S = (h3 & 0x0f0f0f0fu) | ((h1 >> 2) & 0x30303030u);
            M = ((h3 >> 4) & 0x0f0f0f0fu) | ((h2 >> 2) & 0x30303030u);
        }
        const uint32_t sh16 = (q & 1) * 16;
        S >>= sh16;
        M >>= sh16;
        const float d = half_lo(h0);
        const float dmin = half_hi(h0);
        const uint32_t Q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s0 = dot4_u8(opaque(Q[i] & 0x0f0f0f0fu), xv.lo[i], s0);
            s1 = dot4_u8(opaque(Q[i] & 0xf0f0f0f0u), xv.hi[i], s1);
        }
        const float r0 = d * ubyte0(S) * s0 - dmin * ubyte0(M) * xv.sl;
        const float r1 = d * (ubyte1(S) * 0.0625f) * s1 - dmin * ubyte1(M) * xv.sh;
        return r0 + r1;
    }
};

// Q6_K: lane q = (n, h) (n = q >> 1, h = q & 1) of a super-block takes ql
// bytes [64n + 16h, +16) and [64n + 32 + 16h, +16) and qh bytes
// [32n + 16h, +16): quarter t (0..3) gives elements 128n + 32t + 16h + i,
// low nibbles of the first / second ql slice for t = 0 / 1, high nibbles for
// t = 2 / 3, qh bits 2t, 2t + 1, scale sc[8n + h + 2t] (model.cpp:646-683).
template <>
struct Slice<kQ6_K> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 210;
    struct X {
        float4 v[4][4];
        float s[4];
    };
    __device__ static __forceinline__ X load_x(const float* x, const float* xs16, uint32_t q) {
        const uint32_t n = q >> 1, h = q & 1;
        X v;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t e0 = 128 * n + 32 * t + 16 * h;
#pragma unroll
            for (int i = 0; i < 4; ++i) v.v[t][i] = ldx4(x + e0 + 4 * i);
            v.s[t] = 32.0f * xs16[e0 >> 4];
        }
        return v;
    }
    struct W {
        uint4 l0, l1, qh;
        uint32_t sc;  // sc[8n + h + 2t] in byte t
        uint32_t d;
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t q) {
        const uint32_t n = q >> 1, h = q & 1;
        W w;
        w.l0 = ld128_a2(u + 64 * n + 16 * h);
        w.l1 = ld128_a2(u + 64 * n + 32 + 16 * h);
        w.qh = ld128_a2(u + 128 + 32 * n + 16 * h);
        // scales 8n .. 8n + 7 and d (bytes 192 + 8n .. and 208).
        const uint32_t ts = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(u + 192 + 8 * n) & 3u);
        const uint8_t* tb = u + 192 + 8 * n - ts;
        const uint32_t a = *reinterpret_cast<const uint32_t*>(tb);
        const uint32_t b = *reinterpret_cast<const uint32_t*>(tb + 4);
        const uint32_t c = *reinterpret_cast<const uint32_t*>(tb + 8);
        const uint32_t lo = __builtin_amdgcn_alignbyte(b, a, ts);  // sc[8n .. 8n + 3]
        const uint32_t hi = __builtin_amdgcn_alignbyte(c, b, ts);  // sc[8n + 4 .. 8n + 7]
        const uint32_t sh = 8 * h;
        w.sc = ((lo >> sh) & 0xffu) | (((lo >> (sh + 16)) & 0xffu) << 8) | (((hi >> sh) & 0xffu) << 16) |
               (((hi >> (sh + 16)) & 0xffu) << 24);
        w.d = load_u16_a2(u + 208);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t, const X& xv) {
        const uint32_t L0[4] = {w.l0.x, w.l0.y, w.l0.z, w.l0.w};
        const uint32_t L1[4] = {w.l1.x, w.l1.y, w.l1.z, w.l1.w};
        const uint32_t H[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t t0 = (L0[i] & 0x0f0f0f0fu) | ((H[i] << 4) & 0x30303030u);
            const uint32_t t1 = (L1[i] & 0x0f0f0f0fu) | ((H[i] << 2) & 0x30303030u);
            const uint32_t t2 = ((L0[i] >> 4) & 0x0f0f0f0fu) | (H[i] & 0x30303030u);
            const uint32_t t3 = ((L1[i] >> 4) & 0x0f0f0f0fu) | ((H[i] >> 2) & 0x30303030u);
            s[0] = dot4_u8(opaque(t0), xv.v[0][i], s[0]);
            s[1] = dot4_u8(opaque(t1), xv.v[1][i], s[1]);
            s[2] = dot4_u8(opaque(t2), xv.v[2][i], s[2]);
            s[3] = dot4_u8(opaque(t3), xv.v[3][i], s[3]);
        }
        const float d = half_lo(w.d);
        float r = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float sc = static_cast<float>(static_cast<int8_t>((w.sc >> (8 * t)) & 0xffu));
            r += d * sc * (s[t] - xv.s[t]);
        }
        return r;
    }
};

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
    return v;
}

constexpr uint32_t kSliceMaxRows = 64;  // rows per block
constexpr uint32_t kSliceMaxWaves = 8;

template <uint32_t T, int R, int MODE>
__global__ __launch_bounds__(512) void gemv_slice_kernel(const uint8_t* __restrict__ w,
                                                         const uint8_t* __restrict__ w2, size_t row_bytes,
                                                         const float* __restrict__ x, const float* __restrict__ xs16,
                                                         const float* __restrict__ bias,
                                                         const float* __restrict__ residual, float* __restrict__ y,
                                                         float* __restrict__ ys16, uint32_t n, uint32_t units,
                                                         uint32_t wpr, uint32_t teams, uint32_t rpb) {
    using S = Slice<T>;
    constexpr int NR = MODE == 1 ? 2 * R : R;
    __shared__ float part[kSliceMaxWaves][(MODE == 1 ? 2 : 1) * kSliceMaxRows];
    __shared__ float outs[kSliceMaxRows];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t team = wave / wpr, ks = wave % wpr;
    const uint32_t q = lane & 3, slot = lane >> 2;
    const uint32_t u = ks * 16 + slot;
    const bool active = u < units;
    const uint32_t uu = active ? u : units - 1;  // idle lanes load a valid unit and contribute 0
    const typename S::X xv = S::load_x(x + static_cast<size_t>(uu) * S::elems, xs16 + uu * (S::elems / 16), q);
    const uint32_t r0 = blockIdx.x * rpb;
    const uint32_t r1 = min(n, r0 + rpb);

    // Software pipeline: the next R rows' weights are in flight while the
    // current R rows are multiplied and reduced.
    const uint32_t step = teams * R;
    typename S::W cur[NR], nxt[NR];
    auto load_rows = [&](uint32_t base, typename S::W* dst) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const size_t row = min(base + i, n - 1);
            dst[i] = S::load_w(w + row * row_bytes + static_cast<size_t>(uu) * S::bytes, q);
            if (MODE == 1) dst[R + i] = S::load_w(w2 + row * row_bytes + static_cast<size_t>(uu) * S::bytes, q);
        }
    };
    uint32_t rr = r0 + team * R;
    if (rr < r1) load_rows(rr, cur);
    for (; rr < r1; rr += step) {
        if (rr + step < r1) load_rows(rr + step, nxt);
        float acc[NR];
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const float v = S::dot(cur[i], q, xv);
            acc[i] = wave_sum64(active ? v : 0.0f);
        }
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                if (rr + i < r1) {
                    part[ks][rr + i - r0] = acc[i];
                    if (MODE == 1) part[ks][kSliceMaxRows + rr + i - r0] = acc[R + i];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NR; ++i) cur[i] = nxt[i];
    }
    __syncthreads();
    for (uint32_t t = tid; t < r1 - r0; t += blockDim.x) {
        float s = 0.0f;
        for (uint32_t k = 0; k < wpr; ++k) s += part[k][t];
        if (MODE == 0) {
            if (bias) s += bias[r0 + t];
            if (residual) s += residual[r0 + t];
            y[r0 + t] = s;
        } else {
            float up = 0.0f;
            for (uint32_t k = 0; k < wpr; ++k) up += part[k][kSliceMaxRows + t];
            const float v = silu_mul(s, up);
            y[r0 + t] = v;
            outs[t] = v;
        }
    }
    if (MODE == 1 && ys16) {
        __syncthreads();
        for (uint32_t g = tid; g < (r1 - r0) / 16; g += blockDim.x) {
            float t = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) t += outs[16 * g + i];
            ys16[(r0 + 16 * g) / 16] = t;
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

// Tiling code: 10 * R + OPR.
constexpr int kTilings[] = {11, 12, 14, 18, 21, 22, 24, 28, 41, 42, 44, 48};

template <uint32_t T, int MODE>
int launch_typed(int tiling, const void* w, const void* w2, size_t row_bytes, const float* x, const float* xs16,
                 const float* bias, const float* residual, float* y, float* ys16, uint32_t n, uint32_t units,
                 hipStream_t stream, const Batch& batch = Batch(), uint32_t vectors = 1) {
    const auto* wp = static_cast<const uint8_t*>(w);
    const auto* wp2 = static_cast<const uint8_t*>(w2);
    const int R = tiling / 10, OPR = tiling % 10;
    const uint32_t rpb = 32u * R / OPR;
    const dim3 grid((n + rpb - 1) / rpb, vectors);
    switch (tiling) {
#define HIPLLM_GEMV_CASE(RR, OO)                                                                           \
    case 10 * RR + OO:                                                                                     \
        hipLaunchKernelGGL((gemv_kernel<T, RR, OO, MODE>), grid, dim3(256), 0, stream, wp, wp2, row_bytes, \
                           x, xs16, bias, residual, y, ys16, n, units, batch);                             \
        break;
        HIPLLM_GEMV_CASE(1, 1)
        HIPLLM_GEMV_CASE(1, 2)
        HIPLLM_GEMV_CASE(1, 4)
        HIPLLM_GEMV_CASE(1, 8)
        HIPLLM_GEMV_CASE(2, 1)
        HIPLLM_GEMV_CASE(2, 2)
        HIPLLM_GEMV_CASE(2, 4)
        HIPLLM_GEMV_CASE(2, 8)
        HIPLLM_GEMV_CASE(4, 1)
        HIPLLM_GEMV_CASE(4, 2)
        HIPLLM_GEMV_CASE(4, 4)
        HIPLLM_GEMV_CASE(4, 8)
#undef HIPLLM_GEMV_CASE
    default:
        return kInvalidArgument;
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

// Slice-form codes: 2000 + 100 R + 10 teams + rpb / 16, with R in {2, 4},
// teams in {1, 2, 4, 8}, rows per block rpb in {16, 32, 48, 64}.
struct SliceCfg {
    int R;
    uint32_t teams, rpb;
};

bool decode_slice(int code, SliceCfg& cfg) {
    if (code < 2000 || code > 2999) return false;
    cfg.R = (code / 100) % 10;
    cfg.teams = static_cast<uint32_t>((code / 10) % 10);
    cfg.rpb = 16u * static_cast<uint32_t>(code % 10);
    return (cfg.R == 2 || cfg.R == 4) && (cfg.teams == 1 || cfg.teams == 2 || cfg.teams == 4 || cfg.teams == 8) &&
           cfg.rpb >= 16 && cfg.rpb <= kSliceMaxRows;
}

template <uint32_t T, int MODE>
int launch_slice(const SliceCfg& cfg, const void* w, const void* w2, size_t row_bytes, const float* x,
                 const float* xs16, const float* bias, const float* residual, float* y, float* ys16, uint32_t n,
                 uint32_t units, hipStream_t stream) {
    const uint32_t wpr = (units + 15) / 16;
    if (wpr * cfg.teams > kSliceMaxWaves) return kInvalidArgument;
    const dim3 grid((n + cfg.rpb - 1) / cfg.rpb);
    const dim3 block(64 * wpr * cfg.teams);
    const auto* wp = static_cast<const uint8_t*>(w);
    const auto* wp2 = static_cast<const uint8_t*>(w2);
    if (cfg.R == 4) {
        hipLaunchKernelGGL((gemv_slice_kernel<T, 4, MODE>), grid, block, 0, stream, wp, wp2, row_bytes, x, xs16, bias,
                           residual, y, ys16, n, units, wpr, cfg.teams, cfg.rpb);
    } else {
        hipLaunchKernelGGL((gemv_slice_kernel<T, 2, MODE>), grid, block, 0, stream, wp, wp2, row_bytes, x, xs16, bias,
                           residual, y, ys16, n, units, wpr, cfg.teams, cfg.rpb);
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

bool slice_type(uint32_t type) { return type == kQ4_K || type == kQ6_K; }

// Measured choice on MI355X (tests sweep every code; these won per shape):
// Q4_K keeps the octet form (R = 4 or 2, OPR = 8) up to tens of thousands of
// rows and switches to the slice form for LM-head-sized matrices; Q6_K, with
// more bit work per byte, prefers the slice form once rows hold >= 12
// super-blocks.
int gemv_pick_shape(uint32_t type, uint32_t n, uint32_t units, int mode) {
    if (type == kQ4_K) {
        if (mode == 0 && n >= 65536 && units >= 12) return 2411;
        return units >= 32 ? 28 : 48;
    }
    if (type == kQ6_K && units >= 12) {
        if (n >= 65536) return mode == 0 ? 2442 : 2222;
        if (units >= 32) return 2211;
        if (n >= 8192) return 2241;
        return 28;
    }
    return gemv_default_tiling(n, units, mode);
}

// The fused SwiGLU form writes per-16 sums of its outputs, so its octet
// tilings need rows per block (32 R / OPR) divisible by 16.
int gemv_pick(uint32_t type, uint32_t n, uint32_t units, int mode) {
    const int code = gemv_pick_shape(type, n, units, mode);
    if (mode == 1 && code < 100 && (32 * (code / 10) / (code % 10)) % 16 != 0) {
        return gemv_default_tiling(n, units, 1);
    }
    return code;
}

uint32_t unit_elems(uint32_t type) {
    switch (type) {
    case kQ4_K: case kQ6_K: case kF32: case kF16: return 256;
    case kQ8_0: case kQ5_0: return 64;
    default: return 0;
    }
}

bool valid_tiling(int t) {
    for (int v : kTilings) {
        if (v == t) return true;
    }
    return false;
}

}  // namespace

// Default tiling: the largest R and smallest OPR (least activation traffic,
// fewest cross-octet reductions) that still launches >= 1024 waves, with OPR
// chosen so units split evenly across the octets of a row group.
int gemv_default_tiling(uint32_t n, uint32_t units, int mode, uint32_t vectors) {
    const uint32_t target_waves = 1024;
    int best = 0;
    double best_score = -1.0;
    for (int t : kTilings) {
        const int R = t / 10, OPR = t % 10;
        const uint32_t rpb = 32u * R / OPR;
        if (mode == 1 && rpb % 16 != 0) continue;
        const uint32_t blocks = (n + rpb - 1) / rpb;
        const uint32_t waves = blocks * 4 * vectors;
        const uint32_t per = (units + OPR - 1) / OPR;               // units of the busiest octet
        const double balance = static_cast<double>(units) / (per * OPR);
        const double fill = waves >= target_waves ? 1.0 : static_cast<double>(waves) / target_waves;
        // Prefer fill, then balance, then larger R (activation reuse), then smaller OPR.
        const double score = fill * 4.0 + balance * 2.0 + R * 0.05 - OPR * 0.01;
        if (score > best_score) {
            best_score = score;
            best = t;
        }
    }
    return best;
}

int launch_prep_sums(const float* x, float* xs16, size_t k, hipStream_t stream) {
    if (!x || !xs16 || k == 0 || k % 16 != 0) return kInvalidArgument;
    const uint32_t groups = static_cast<uint32_t>(k / 16);
    hipLaunchKernelGGL(prep_sums_kernel, dim3((groups + 255) / 256), dim3(256), 0, stream, x, xs16, groups);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

// GEMV over pre-computed xs16. tiling 0 selects the default.
int launch_gemv_prepped(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* xs16,
                        const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                        hipStream_t stream) {
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
    const uint32_t nn = static_cast<uint32_t>(n);
    SliceCfg sc;
    const int code = tiling ? tiling : gemv_pick(type, nn, units, 0);
    if (decode_slice(code, sc)) {
        if (!slice_type(type)) return kInvalidArgument;
        if (type == kQ4_K) return launch_slice<kQ4_K, 0>(sc, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
        return launch_slice<kQ6_K, 0>(sc, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    }
    if (!valid_tiling(code)) return kInvalidArgument;
    const int t = code;
    switch (type) {
    case kQ4_K: return launch_typed<kQ4_K, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    case kQ6_K: return launch_typed<kQ6_K, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    case kQ8_0: return launch_typed<kQ8_0, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    case kQ5_0: return launch_typed<kQ5_0, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    case kF32: return launch_typed<kF32, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
    case kF16: return launch_typed<kF16, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream);
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
    if ((type == kF32 || type == kF16) &&
        (row_bytes % 16 != 0 || reinterpret_cast<uintptr_t>(wg) % 16 != 0 || reinterpret_cast<uintptr_t>(wu) % 16 != 0)) {
        return kInvalidArgument;
    }
    if (reinterpret_cast<uintptr_t>(wg) % 2 != 0 || reinterpret_cast<uintptr_t>(wu) % 2 != 0 || row_bytes % 2 != 0) {
        return kInvalidArgument;
    }
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return kInvalidArgument;
    if (ys16 && n % 16 != 0) return kInvalidArgument;
    if (n > 0x7fffffffu || k > 0x7fffffffu) return kLengthError;
    const uint32_t units = static_cast<uint32_t>(k / ue);
    const uint32_t nn = static_cast<uint32_t>(n);
    SliceCfg sc;
    const int code = gemv_pick(type, nn, units, 1);
    if (decode_slice(code, sc)) {
        if (type == kQ4_K) return launch_slice<kQ4_K, 1>(sc, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
        return launch_slice<kQ6_K, 1>(sc, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    }
    const int t = code;
    switch (type) {
    case kQ4_K: return launch_typed<kQ4_K, 1>(t, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    case kQ6_K: return launch_typed<kQ6_K, 1>(t, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    case kQ8_0: return launch_typed<kQ8_0, 1>(t, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    case kQ5_0: return launch_typed<kQ5_0, 1>(t, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    case kF32: return launch_typed<kF32, 1>(t, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    case kF16: return launch_typed<kF16, 1>(t, wg, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream);
    default: return kInvalidArgument;
    }
}

}  // namespace hipllm

namespace hipllm {

// A batch of GEMVs through one matrix or through routed experts (see Batch):
// vector j computes y[j, :n] = W_j x_j (+ bias) (+ residual[j]) or, with
// wu != nullptr, y[j] = silu(Wg_j x_j) * (Wu_j x_j) with optional ys16[j].
int launch_gemv_batched(uint32_t type, const void* w, const void* wu, size_t row_bytes, const float* x,
                        const float* xs16, const float* bias, const float* residual, float* y, float* ys16, size_t n,
                        size_t k, size_t vectors, const int32_t* ids, size_t experts, size_t routes,
                        size_t expert_stride, int x_routed, size_t ldx, size_t ldy, hipStream_t stream) {
    const uint32_t ue = unit_elems(type);
    if (!w || !x || !xs16 || !y || n == 0 || k == 0 || ue == 0 || k % ue != 0 || vectors == 0) {
        return kInvalidArgument;
    }
    if (row_bytes < k / block_elems(type) * block_bytes(type)) return kInvalidArgument;
    const bool need16 = type == kQ4_K || type == kF32 || type == kF16;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w), ua = reinterpret_cast<uintptr_t>(wu);
    if (need16 && (row_bytes % 16 != 0 || wa % 16 != 0 || (wu && ua % 16 != 0) || expert_stride % 16 != 0)) {
        return kInvalidArgument;
    }
    if (wa % 2 != 0 || (wu && ua % 2 != 0) || row_bytes % 2 != 0 || expert_stride % 2 != 0) return kInvalidArgument;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || ldx < k || ldx % 16 != 0 || ldy < n) return kInvalidArgument;
    if (ids && (experts == 0 || routes == 0 || expert_stride < n * row_bytes)) return kInvalidArgument;
    if (!ids && (routes == 0)) return kInvalidArgument;
    if (ys16 && (n % 16 != 0 || ldy % 16 != 0)) return kInvalidArgument;
    if (n > 0x7fffffffu || k > 0x7fffffffu || vectors > 65535 || ldx > 0xffffffffu || ldy > 0xffffffffu ||
        experts > 0xffffffffu || routes > 0xffffffffu) {
        return kLengthError;
    }
    Batch b;
    b.ids = ids;
    b.experts = ids ? static_cast<uint32_t>(experts) : 1u;
    b.routes = static_cast<uint32_t>(routes);
    b.expert_stride = ids ? expert_stride : 0;
    b.x_routed = x_routed ? 1u : 0u;
    b.ldx = static_cast<uint32_t>(ldx);
    b.ldy = static_cast<uint32_t>(ldy);
    const uint32_t units = static_cast<uint32_t>(k / ue);
    const uint32_t nn = static_cast<uint32_t>(n);
    const uint32_t nv = static_cast<uint32_t>(vectors);
    if (!wu) {
        int t = gemv_default_tiling(nn, units, 0, nv);
        switch (type) {
        case kQ4_K: return launch_typed<kQ4_K, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream, b, nv);
        case kQ6_K: return launch_typed<kQ6_K, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream, b, nv);
        case kQ8_0: return launch_typed<kQ8_0, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream, b, nv);
        case kQ5_0: return launch_typed<kQ5_0, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream, b, nv);
        case kF32: return launch_typed<kF32, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream, b, nv);
        case kF16: return launch_typed<kF16, 0>(t, w, nullptr, row_bytes, x, xs16, bias, residual, y, nullptr, nn, units, stream, b, nv);
        default: return kInvalidArgument;
        }
    }
    if (bias || residual) return kInvalidArgument;
    const int t = gemv_default_tiling(nn, units, 1, nv);
    switch (type) {
    case kQ4_K: return launch_typed<kQ4_K, 1>(t, w, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream, b, nv);
    case kQ6_K: return launch_typed<kQ6_K, 1>(t, w, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream, b, nv);
    case kQ8_0: return launch_typed<kQ8_0, 1>(t, w, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream, b, nv);
    case kQ5_0: return launch_typed<kQ5_0, 1>(t, w, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream, b, nv);
    case kF32: return launch_typed<kF32, 1>(t, w, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream, b, nv);
    case kF16: return launch_typed<kF16, 1>(t, w, wu, row_bytes, x, xs16, nullptr, nullptr, y, ys16, nn, units, stream, b, nv);
    default: return kInvalidArgument;
    }
}

}  // namespace hipllm
