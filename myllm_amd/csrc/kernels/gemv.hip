// Decode GEMV over native GGUF block-quantized weights: y[N] = W[N,K] x[K].
//
// Replaces the reference's one-thread-per-row GEVMs (metal_llm.metal:708-781,
// dot_q*_f32 319-553; host encode_vector_product metal_llm.mm:1891-1999) with
// a wave-cooperative, integer-dot design for CDNA4:
//
// * An "octet" of 8 lanes owns one unit of a row (a 256-value super-block for
//   Q4_K / Q6_K / F32 / F16, four 32-value blocks for Q8_0 / Q5_0). Every lane
//   issues 128-bit loads of its slice of the unit, so eight lanes read one
//   contiguous unit.
// * Each octet computes R rows at once: a lane loads its activation slice of a
//   unit once and multiplies it into the same slice of R rows.
// * OPR octets share a row group and split its units round-robin (K split);
//   up to 8 of them sit in one wave (shuffle reduction), 16 or 32 span 2 or 4
//   waves (then wave partials meet in LDS). A block is 4 waves, 32 octets,
//   32 / OPR row groups of R rows.
// * Quantized weights multiply the XGroup form of the activation (common.h):
//   per 16 values, 24-bit fixed point in three signed-byte digits. A weight
//   quant dword (4 quants as bytes) times a digit dword is one v_dot4_i32_i8,
//   exact in integers, so a 16-value slice costs 3 dot4 per 4 quants plus the
//   nibble / bit unpacking, about 1.5 VALU instructions per weight instead of
//   the 4+ of a convert-to-float multiply-add. The three digit sums combine
//   into one FP32 value per 16-group, scaled by the group's e and by the
//   block's FP32 scales; the constant part of each affine format (Q4_K's
//   -dmin*m, Q6_K's -32, Q5_0's -16) uses the group's FP32 sum. F32 / F16
//   weights multiply the FP32 activation directly.
// * Partials reduce with lane shuffles in a fixed order (deterministic); the
//   epilogue adds bias and residual, or applies SwiGLU for the fused gate/up
//   form and writes the XGroup form of its output for the down projection.
//
// Weight rows may be only 2-byte aligned (Q6_K / Q8_0 / Q5_0 block sizes are
// 210 / 34 / 22 bytes); such loads read the enclosing aligned dwords and
// realign with v_alignbyte. Device weight buffers carry 256 bytes of tail
// padding so those reads stay in bounds.
#include "common.h"
#include "launch.h"
#include "norm.h"
#include "router.h"

namespace hipllm {

namespace {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4a16 __attribute__((ext_vector_type(4)));

// Weight loads. Ordinary cached loads: several lanes and instructions touch
// each cache line of a block (headers, scales, realigned tails), which
// nontemporal loads would send to memory again (measured slower on MI355X).
__device__ __forceinline__ uint4 ldw128(const uint8_t* p) {  // 16-byte aligned
    const u32x4a16 v = *reinterpret_cast<const u32x4a16*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Streaming loads of bytes that exactly one lane of one wave reads (the x16
// form's quant slices, each 16-byte piece read once per launch).
__device__ __forceinline__ uint4 ldw128_nt(const uint8_t* p) {  // 16-byte aligned
    const u32x4a16 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4a16*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint4 ldw128_a4(const uint8_t* p) {  // 4-byte aligned
    const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t ldw32(const uint8_t* p) {  // 4-byte aligned
    return *reinterpret_cast<const uint32_t*>(p);
}

__device__ __forceinline__ uint32_t ldw16(const uint8_t* p) {  // 2-byte aligned
    return *reinterpret_cast<const uint16_t*>(p);
}

// 16 bytes at a 2-byte-aligned address p, fetched as the 20 enclosing
// dword-aligned bytes; realign() extracts them once the load has landed
// (realigning at load time would make every load wait for its data).
// Pointer arithmetic (not integer casts) keeps the global address space.
struct Raw20 {
    uint4 v;
    uint32_t e;
};

__device__ __forceinline__ uint32_t misalign(const uint8_t* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
}

__device__ __forceinline__ Raw20 ldw_raw20(const uint8_t* p) {
    const uint8_t* base = p - misalign(p);
    Raw20 r;
    r.v = ldw128_a4(base);
    r.e = ldw32(base + 16);
    return r;
}

// 20 bytes at a 2-byte-aligned address (24 enclosing bytes).
struct Raw24 {
    uint4 v;
    uint32_t e0, e1;
};

typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ Raw24 ldw_raw24(const uint8_t* p) {
    const uint8_t* base = p - misalign(p);
    Raw24 r;
    r.v = ldw128_a4(base);
    const u32x2a4 t = *reinterpret_cast<const u32x2a4*>(base + 16);
    r.e0 = t.x;
    r.e1 = t.y;
    return r;
}

__device__ __forceinline__ uint4 realign(const Raw20& r, uint32_t s) {
    return make_uint4(__builtin_amdgcn_alignbyte(r.v.y, r.v.x, s), __builtin_amdgcn_alignbyte(r.v.z, r.v.y, s),
                      __builtin_amdgcn_alignbyte(r.v.w, r.v.z, s), __builtin_amdgcn_alignbyte(r.e, r.v.w, s));
}

__device__ __forceinline__ float4 ldx4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// One XGroup in registers. All 16 dwords are used: a load whose unused
// lanes the register allocator recycles would stall on the load in flight.
struct XG {
    uint32_t s0[4], s1[4], s2[4];
    float sum, e, e256, e65536;
};

__device__ __forceinline__ XG ldxg(const XGroup* g) {
    const uint4* p = reinterpret_cast<const uint4*>(g);
    const uint4 a = p[0], b = p[1], c = p[2], m = p[3];
    XG v;
    v.s0[0] = a.x, v.s0[1] = a.y, v.s0[2] = a.z, v.s0[3] = a.w;
    v.s1[0] = b.x, v.s1[1] = b.y, v.s1[2] = b.z, v.s1[3] = b.w;
    v.s2[0] = c.x, v.s2[1] = c.y, v.s2[2] = c.z, v.s2[3] = c.w;
    v.sum = __uint_as_float(m.x);
    v.e = __uint_as_float(m.y);
    v.e256 = __uint_as_float(m.z);
    v.e65536 = __uint_as_float(m.w);
    return v;
}

// Digit sums of 4 quants (signed bytes of q) against dword i of a group.
struct Acc3 {
    int a0 = 0, a1 = 0, a2 = 0;
};

__device__ __forceinline__ void dot3(uint32_t q, const XG& x, int i, Acc3& s) {
    s.a0 = __builtin_amdgcn_sdot4(static_cast<int>(q), static_cast<int>(x.s0[i]), s.a0, false);
    s.a1 = __builtin_amdgcn_sdot4(static_cast<int>(q), static_cast<int>(x.s1[i]), s.a1, false);
    s.a2 = __builtin_amdgcn_sdot4(static_cast<int>(q), static_cast<int>(x.s2[i]), s.a2, false);
}

// e * sum(q * x_int) of a 16-group as FP32: the digit sums (each below 2^24
// in magnitude, so converted exactly) weighted by e, 256 e and 65536 e.
__device__ __forceinline__ float dot3_value(const Acc3& s, const XG& x) {
    return fmaf(static_cast<float>(s.a2), x.e65536, fmaf(static_cast<float>(s.a1), x.e256, static_cast<float>(s.a0) * x.e));
}

// Value of lane I of this lane's quad (DPP quad_perm broadcast). All four
// lanes of a quad are always active together (they belong to one octet), so
// no "old" value is needed.
template <int I>
__device__ __forceinline__ uint32_t quad_lane(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), I * 0x55, 0xf, 0xf, true));
}

template <uint32_t T>
struct Unit;

// Q4_K: 144-byte super-block {d, dmin, scales[12], qs[128]}. Lane c of the
// octet takes qs bytes [16c, 16c+16): j = c/2, l0 = 16 (c & 1); its low
// nibbles are elements 64j+l0.. of sub-block 2j (16-group 4j + (c & 1)), its
// high nibbles elements 64j+32+l0.. of sub-block 2j+1 (16-group 4j + 2 +
// (c & 1)) (model.cpp:616-644).
template <>
struct Unit<kQ4_K> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 144;
    static constexpr bool ragged = false;
    struct X {
        XG a, b;
    };
    __device__ static __forceinline__ X load_x(const float*, const XGroup* xq, uint32_t c) {
        const uint32_t g = 4 * (c >> 1) + (c & 1);
        X v;
        v.a = ldxg(xq + g);
        v.b = ldxg(xq + g + 2);
        return v;
    }
    struct W {
        uint32_t head;  // header dword (c & 3)
        uint4 q;
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        W w;
        w.head = ldw32(u + 4 * (c & 3));
        w.q = ldw128(u + 16 + 16 * c);
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
        const uint32_t Q[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        Acc3 sa, sb;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            dot3(Q[i] & 0x0f0f0f0fu, xv.a, i, sa);
            dot3((Q[i] >> 4) & 0x0f0f0f0fu, xv.b, i, sb);
        }
        const float fa = dot3_value(sa, xv.a);
        const float fb = dot3_value(sb, xv.b);
        return (d * ubyte0(S) * fa - dmin * ubyte0(M) * xv.a.sum) + (d * ubyte1(S) * fb - dmin * ubyte1(M) * xv.b.sum);
    }
};

// Q6_K: 210-byte super-block {ql[128], qh[64], scales[16] int8, d}. Lane
// c = (n, m, h) takes ql bytes [64n + 32m + 16h, +16) and qh bytes
// [32n + 16h, +16): its low nibbles are elements 128n + 32m + 16h + l
// (16-group 8n + 2m + h) and its high nibbles elements 128n + 64 + 32m +
// 16h + l (16-group + 4) (model.cpp:646-683), each 16-group with one int8
// scale.
template <>
struct Unit<kQ6_K> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 210;
    static constexpr bool ragged = false;
    struct X {
        XG a, b;
    };
    __device__ static __forceinline__ X load_x(const float*, const XGroup* xq, uint32_t c) {
        const uint32_t n = c >> 2, m = (c >> 1) & 1, hh = c & 1;
        const uint32_t g = 8 * n + 2 * m + hh;
        X v;
        v.a = ldxg(xq + g);
        v.b = ldxg(xq + g + 4);
        return v;
    }
    struct W {
        Raw20 ql, qh, tail;  // tail: scales[16] and d (bytes 192..209)
        uint32_t s;          // misalignment of the super-block (all three share it)
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        const uint32_t n = c >> 2, m = (c >> 1) & 1, hh = c & 1;
        W w;
        w.ql = ldw_raw20(u + 64 * n + 32 * m + 16 * hh);
        w.qh = ldw_raw20(u + 128 + 32 * n + 16 * hh);
        w.tail = ldw_raw20(u + 192);
        w.s = misalign(u);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t c, const X& xv) {
        const uint32_t n = c >> 2, hh = c & 1;
        const uint4 ql = realign(w.ql, w.s), qh = realign(w.qh, w.s);
        const uint4 t = w.tail.v;
        const uint32_t ts = w.s, t4 = w.tail.e;
        const uint32_t sc0_3 = __builtin_amdgcn_alignbyte(t.y, t.x, ts);
        const uint32_t sc4_7 = __builtin_amdgcn_alignbyte(t.z, t.y, ts);
        const uint32_t sc8_11 = __builtin_amdgcn_alignbyte(t.w, t.z, ts);
        const uint32_t sc12_15 = __builtin_amdgcn_alignbyte(t4, t.w, ts);
        // Scale bytes used: index 8n + hh + 2m (low nibbles) and +4 (high).
        const uint32_t m = (c >> 1) & 1;
        const uint32_t wlo = n ? sc8_11 : sc0_3;
        const uint32_t whi = n ? sc12_15 : sc4_7;
        const uint32_t sel = 8 * (hh + 2 * m);
        const uint32_t sc = ((wlo >> sel) & 0xffu) | (((whi >> sel) & 0xffu) << 8);
        const uint32_t dbits = __builtin_amdgcn_alignbyte(t4, t4, ts) & 0xffffu;  // bytes 16..17 of the tail
        const uint32_t shl = 4 - 2 * m;  // qh bits (2m, 2m+1) -> bits 4, 5
        const uint32_t shr = 2 * m;      // qh bits (2m+4, 2m+5) -> bits 4, 5
        const uint32_t L[4] = {ql.x, ql.y, ql.z, ql.w};
        const uint32_t H[4] = {qh.x, qh.y, qh.z, qh.w};
        Acc3 sa, sb;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (L[i] & 0x0f0f0f0fu) | ((H[i] << shl) & 0x30303030u);
            const uint32_t hi = ((L[i] >> 4) & 0x0f0f0f0fu) | ((H[i] >> shr) & 0x30303030u);
            dot3(lo, xv.a, i, sa);
            dot3(hi, xv.b, i, sb);
        }
        const float d = half_lo(dbits);
        const float sA = static_cast<float>(static_cast<int8_t>(sc & 0xffu));
        const float sB = static_cast<float>(static_cast<int8_t>((sc >> 8) & 0xffu));
        // value = d * sc * (q - 32)
        const float fa = fmaf(-32.0f, xv.a.sum, dot3_value(sa, xv.a));
        const float fb = fmaf(-32.0f, xv.b.sum, dot3_value(sb, xv.b));
        return d * sA * fa + d * sB * fb;
    }
};

// Q8_0: four 34-byte blocks {d, qs[32] int8} per unit. Lane c = (b, h) takes
// qs bytes [16h, 16h+16) of block b: elements 32b + 16h + i, 16-group c of
// the unit (model.cpp:603-614).
template <>
struct Unit<kQ8_0> {
    static constexpr uint32_t elems = 128;
    static constexpr uint32_t bytes = 136;
    static constexpr bool ragged = true;
    struct X {
        XG a;
    };
    __device__ static __forceinline__ X load_x(const float*, const XGroup* xq, uint32_t c) {
        X v;
        v.a = ldxg(xq + c);
        return v;
    }
    struct W {
        Raw20 q;
        uint32_t d, s;
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        const uint8_t* blk = u + 34 * (c >> 1);
        const uint8_t* qs = blk + 2 + 16 * (c & 1);
        W w;
        w.d = ldw16(blk);
        w.q = ldw_raw20(qs);
        w.s = misalign(qs);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t, const X& xv) {
        const uint4 q = realign(w.q, w.s);
        const uint32_t Q[4] = {q.x, q.y, q.z, q.w};
        Acc3 s;
#pragma unroll
        for (int i = 0; i < 4; ++i) dot3(Q[i], xv.a, i, s);
        return half_lo(w.d) * dot3_value(s, xv.a);
    }
};

// Q5_0: four 22-byte blocks {d, qh[4], qs[16]} per unit. Lane c = (b, h)
// takes elements 32b + 16h + i: low (h = 0) or high (h = 1) nibbles of qs[i]
// with fifth bit i + 16h of qh (model.cpp:581-601).
template <>
struct Unit<kQ5_0> {
    static constexpr uint32_t elems = 128;
    static constexpr uint32_t bytes = 88;
    static constexpr bool ragged = true;
    struct X {
        XG a;
    };
    __device__ static __forceinline__ X load_x(const float*, const XGroup* xq, uint32_t c) {
        X v;
        v.a = ldxg(xq + c);
        return v;
    }
    struct W {
        Raw24 qs;  // qh[4] and qs[16] are bytes 2..21 of the block
        uint32_t d, s;
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        const uint8_t* blk = u + 22 * (c >> 1);
        W w;
        w.d = ldw16(blk);
        w.qs = ldw_raw24(blk + 2);
        w.s = misalign(blk + 2);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t c, const X& xv) {
        const uint32_t h = c & 1;
        // Bytes 2..21 of the block: qh (4 bytes) then qs (16 bytes).
        const uint32_t sh = w.s;
        const uint32_t qh = __builtin_amdgcn_alignbyte(w.qs.v.y, w.qs.v.x, sh);
        const uint32_t q0 = __builtin_amdgcn_alignbyte(w.qs.v.z, w.qs.v.y, sh);
        const uint32_t q1 = __builtin_amdgcn_alignbyte(w.qs.v.w, w.qs.v.z, sh);
        const uint32_t q2 = __builtin_amdgcn_alignbyte(w.qs.e0, w.qs.v.w, sh);
        const uint32_t q3 = __builtin_amdgcn_alignbyte(w.qs.e1, w.qs.e0, sh);
        const uint32_t Q[4] = {q0, q1, q2, q3};
        const uint32_t bits = qh >> (16 * h);
        Acc3 s;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t nib = (Q[i] >> (4 * h)) & 0x0f0f0f0fu;
            const uint32_t hb = (bits >> (4 * i)) & 0xfu;
            dot3(nib | (((hb * 0x00204081u) & 0x01010101u) << 4), xv.a, i, s);
        }
        return half_lo(w.d) * fmaf(-16.0f, xv.a.sum, dot3_value(s, xv.a));
    }
};

// F32: 256 values (1024 bytes) per unit; lane c takes values [32c, 32c+32).
template <>
struct Unit<kF32> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 1024;
    static constexpr bool ragged = false;
    struct X {
        float4 a[8];
    };
    __device__ static __forceinline__ X load_x(const float* x, const XGroup*, uint32_t c) {
        X v;
#pragma unroll
        for (int i = 0; i < 8; ++i) v.a[i] = ldx4(x + 32 * c + 4 * i);
        return v;
    }
    struct W {
        uint4 w[8];
    };
    __device__ static __forceinline__ W load_w(const uint8_t* u, uint32_t c) {
        W w;
#pragma unroll
        for (int i = 0; i < 8; ++i) w.w[i] = ldw128(u + 128 * c + 16 * i);
        return w;
    }
    __device__ static __forceinline__ float dot(const W& w, uint32_t, const X& xv) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s = fmaf(__uint_as_float(w.w[i].x), xv.a[i].x, s);
            s = fmaf(__uint_as_float(w.w[i].y), xv.a[i].y, s);
            s = fmaf(__uint_as_float(w.w[i].z), xv.a[i].z, s);
            s = fmaf(__uint_as_float(w.w[i].w), xv.a[i].w, s);
        }
        return s;
    }
};

// F16: 256 values (512 bytes) per unit; lane c takes values [32c, 32c+32).
template <>
struct Unit<kF16> {
    static constexpr uint32_t elems = 256;
    static constexpr uint32_t bytes = 512;
    static constexpr bool ragged = false;
    struct X {
        float4 a[8];
    };
    __device__ static __forceinline__ X load_x(const float* x, const XGroup*, uint32_t c) {
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
        for (int i = 0; i < 4; ++i) w.h[i] = ldw128(u + 64 * c + 16 * i);
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
// ROUTE kernels pick the experts themselves: every block runs the router's
// softmax / top-k / renormalisation (router.h) on its token's logits with its
// first wave, takes its route's expert from LDS, and the first block of each
// token stores the ids and weights (ids_out, weights_out) for the launches
// that follow.
struct Batch {
    const int32_t* ids = nullptr;
    uint32_t experts = 1;
    uint32_t routes = 1;
    size_t expert_stride = 0;
    uint32_t x_routed = 0;
    uint32_t ldx = 0;  // values between input rows (multiple of 16)
    uint32_t ldy = 0;  // values between output rows
    const float* logits = nullptr;  // ROUTE: [tokens, ld_logits] router logits
    uint32_t ld_logits = 0;
    int32_t* ids_out = nullptr;     // ROUTE: [tokens, routes]
    float* weights_out = nullptr;   // ROUTE: [tokens, routes]
};
constexpr uint32_t kRouteMaxExperts = 256;  // logits held 4 per lane by one wave

// MODE 2 epilogue, the MoE combine of one token on the shared expert's down
// projection: y[r] = residual[r] + (sum_q weights[q] down[q n + r] +
// sigmoid(sgate[0]) (W x)[r]), the same operations in the same order as the
// combine kernel.
struct MoeCombine {
    const float* down = nullptr;
    const float* weights = nullptr;
    const float* sgate = nullptr;
    uint32_t routes = 0;
};

constexpr uint32_t kCombineRoutes = 8;  // routes the epilogue loads at once

__device__ __forceinline__ float combine_row(const MoeCombine& m, const float* residual, float shared, uint32_t r,
                                             uint32_t n) {
    // Every route's value is loaded before the sum (in route order).
    float dv[kCombineRoutes], wv[kCombineRoutes];
#pragma unroll
    for (uint32_t q = 0; q < kCombineRoutes; ++q) {
        if (q < m.routes) {
            dv[q] = m.down[static_cast<size_t>(q) * n + r];
            wv[q] = m.weights[q];
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < kCombineRoutes; ++q) {
        if (q < m.routes) acc += wv[q] * dv[q];
    }
    float moe = acc;
    moe += shared * sigmoid_ref(m.sgate[0]);
    return residual[r] + moe;
}

// R rows per octet, OPR octets per row group (K split), 32 / OPR row groups
// per block of 4 waves: rows per block = 32 R / OPR.
// MODE 0: y = W x (+ bias) (+ residual).
// MODE 1: y = silu(W x) * (W2 x); each octet carries R rows of W and the same
//         R rows of W2. yq (optional) receives the XGroup form of y.
// Sum over the OPW octets (8 OPW lanes) of each row group in the wave; the
// group's first lane holds the result. Octet sums by DPP (neighbour swaps,
// then the half-row mirror), 16-lane sums by the row mirror, 32- and 64-lane
// sums from the four row results read with v_readlane.
template <int OPW>
__device__ __forceinline__ float octet_group_sum(float v, uint32_t lane) {
    v += dpp_f32<kDppQuadXor1>(v);
    v += dpp_f32<kDppQuadXor2>(v);
    v += dpp_f32<kDppHalfMirror>(v);
    if constexpr (OPW >= 2) v += dpp_f32<kDppMirror>(v);
    if constexpr (OPW == 4) {
        const float lo = lane_f32(v, 0) + lane_f32(v, 16), hi = lane_f32(v, 32) + lane_f32(v, 48);
        v = lane < 32 ? lo : hi;
    }
    if constexpr (OPW == 8) v = (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
    return v;
}

// NORM (single vector): x is the raw row and gamma its RMSNorm gain; every
// block normalises x into LDS (the XGroup form for quantized weights, FP32
// values for F32 weights; the same bits as the standalone RMSNorm kernel)
// while its first weight loads are in flight, then multiplies from LDS.
// Saves the norm's own launch.
constexpr uint32_t kNormMaxGroups = 512;  // rows of up to 8192 values

// The work of block (bx, by) of a GEMV launch; the kernels below call it with
// their block index (or, for a grouped launch, the index within their job).
template <uint32_t T, int R, int OPR, int MODE, bool NORM, bool ROUTE = false>
__device__ __forceinline__ void gemv_block(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                                           size_t row_bytes, const float* __restrict__ x,
                                           const XGroup* __restrict__ xq, const float* __restrict__ bias,
                                           const float* __restrict__ residual, float* __restrict__ y,
                                           XGroup* __restrict__ yq, uint32_t n, uint32_t units, uint32_t kblocks,
                                           const Batch& batch, const float* __restrict__ gamma, float eps,
                                           uint32_t bx, uint32_t by, const MoeCombine& cmb = MoeCombine()) {
    using U = Unit<T>;
    {
        // Vector j of the batch: shift weights, input, output and residual.
        const uint32_t j = by;
        const uint32_t xrow = batch.x_routed ? j : j / batch.routes;
        if constexpr (ROUTE) {
            __shared__ int32_t route_id[8];
            __shared__ float route_w[8];
            const uint32_t t = j / batch.routes, q = j % batch.routes;
            if (threadIdx.x < 64) {
                topk_row<kRouteMaxExperts / 64>(batch.logits + static_cast<size_t>(t) * batch.ld_logits,
                                                 batch.experts, batch.routes, route_id, route_w, threadIdx.x);
            }
            __syncthreads();
            if (bx == 0 && q == 0 && threadIdx.x < batch.routes) {
                batch.ids_out[t * batch.routes + threadIdx.x] = route_id[threadIdx.x];
                batch.weights_out[t * batch.routes + threadIdx.x] = route_w[threadIdx.x];
            }
            const uint32_t e = min(static_cast<uint32_t>(route_id[q]), batch.experts - 1);
            w += static_cast<size_t>(e) * batch.expert_stride;
            if (MODE == 1) w2 += static_cast<size_t>(e) * batch.expert_stride;
        } else if (batch.ids) {
            const uint32_t e = min(static_cast<uint32_t>(batch.ids[j]), batch.experts - 1);
            w += static_cast<size_t>(e) * batch.expert_stride;
            if (MODE == 1) w2 += static_cast<size_t>(e) * batch.expert_stride;
        }
        x += static_cast<size_t>(xrow) * batch.ldx;
        xq += static_cast<size_t>(xrow) * (batch.ldx / 16);
        y += static_cast<size_t>(j) * batch.ldy;
        if (residual) residual += static_cast<size_t>(j) * batch.ldy;
        if (yq) yq += static_cast<size_t>(j) * (batch.ldy / 16);
    }
    static_assert(OPR == 1 || OPR == 2 || OPR == 4 || OPR == 8 || OPR == 16 || OPR == 32, "OPR");
    constexpr int NR = MODE == 1 ? 2 * R : R;
    constexpr int OPW = OPR < 8 ? OPR : 8;      // octets of a row group inside one wave
    constexpr int WPG = OPR > 8 ? OPR / 8 : 1;  // waves per row group
    constexpr int RPB = (32 / OPR) * R;         // rows per block
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t o = tid >> 3, c = tid & 7;
    const uint32_t rg = o / OPR, slot = o % OPR;
    const uint32_t lrow0 = rg * R;  // first row of this octet within the block
    const uint32_t row0 = bx * RPB + lrow0;

    // Byte offsets of this octet's rows (rows past n are computed, never stored).
    uint32_t roff[R];
#pragma unroll
    for (int i = 0; i < R; ++i) roff[i] = min(row0 + i, n - 1) * static_cast<uint32_t>(row_bytes);
    float acc[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) acc[i] = 0.0f;

    // Ragged last unit (Q8_0 / Q5_0 rows whose block count is not a multiple
    // of 4): lanes past the row read block 0 of the unit and contribute 0.
    auto lane_ok = [&](uint32_t u) { return !U::ragged || 4 * u + (c >> 1) < kblocks; };
    auto load = [&](uint32_t u, typename U::W (&wv)[NR]) {
        const uint32_t ce = lane_ok(u) ? c : (c & 1);
        const uint32_t uo = u * U::bytes;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            wv[i] = U::load_w(w + (roff[i] + uo), ce);
            if (MODE == 1) wv[R + i] = U::load_w(w2 + (roff[i] + uo), ce);
        }
    };
    auto consume = [&](uint32_t u, const typename U::W (&wv)[NR]) {
        const bool ok = lane_ok(u);
        const uint32_t ce = ok ? c : (c & 1);
        const typename U::X xv =
            U::load_x(x + static_cast<size_t>(u) * U::elems, xq + u * (U::elems / 16), ce);
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const float v = U::dot(wv[i], ce, xv);
            acc[i] += ok ? v : 0.0f;
        }
    };
    // One unit per iteration. The tilings that measure fastest give each lane
    // one or two units, so every wave issues all its weight loads at once and
    // latency is covered by the many resident waves (a second register set
    // for prefetching, or staging x in LDS, measured slower: fewer resident
    // waves, extra synchronisation).
    typename U::W wv[NR];
    const bool first = slot < units;
    if (first) load(slot, wv);
    if constexpr (NORM) {
        extern __shared__ __align__(16) uint8_t norm_lds[];  // 4 k bytes, sized at launch
        if constexpr (T == kF32) {
            float* xs = reinterpret_cast<float*>(norm_lds);
            rmsnorm_row_lean(x, gamma, xs, nullptr, kblocks * 32, eps);
            __syncthreads();
            x = xs;
        } else {
            XGroup* xs = reinterpret_cast<XGroup*>(norm_lds);
            if (gamma) {
                rmsnorm_row_lean(x, gamma, nullptr, xs, kblocks * 32, eps);
            } else {
                // No gain: the XGroup form of x itself.
                for (uint32_t g = tid; g < kblocks * 2; g += blockDim.x) xgroup_encode_from(x + 16 * g, xs + g);
            }
            __syncthreads();
            xq = xs;
        }
    }
    if (first) consume(slot, wv);
    for (uint32_t u = slot + OPR; u < units; u += OPR) {
        load(u, wv);
        consume(u, wv);
    }

    // Reduce the 8 lanes of the octet, then the octets of the row group in
    // this wave (DPP inside 16-lane rows, v_readlane across rows).
#pragma unroll
    for (int i = 0; i < NR; ++i) acc[i] = octet_group_sum<OPW>(acc[i], lane);
    __shared__ __align__(16) float outs[RPB];
    const uint32_t blk_row0 = bx * RPB;
    if (WPG == 1) {
        if (c == 0 && slot == 0) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const uint32_t r = row0 + i;
                if (MODE == 2) {
                    if (r < n) y[r] = combine_row(cmb, residual, acc[i], r, n);
                } else if (MODE == 0) {
                    if (r < n) {
                        float s = acc[i];
                        if (bias) s += bias[r];
                        if (residual) s += residual[r];
                        y[r] = s;
                    }
                } else {
                    const float v = r < n ? silu_mul(acc[i], acc[R + i]) : 0.0f;
                    outs[lrow0 + i] = v;
                    if (r < n) y[r] = v;
                }
            }
        }
    } else {
        // Wave partials of each row group meet in LDS, summed in wave order.
        __shared__ float part[4][NR];
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < NR; ++i) part[wave][i] = acc[i];
        }
        __syncthreads();
        if (tid < static_cast<uint32_t>(RPB)) {
            const uint32_t g = tid / R, i = tid % R;
            const uint32_t r = blk_row0 + tid;
            float s = 0.0f, s2 = 0.0f;
#pragma unroll
            for (int k = 0; k < WPG; ++k) {
                s += part[g * WPG + k][i];
                if (MODE == 1) s2 += part[g * WPG + k][R + i];
            }
            if (MODE == 2) {
                if (r < n) y[r] = combine_row(cmb, residual, s, r, n);
            } else if (MODE == 0) {
                if (r < n) {
                    if (bias) s += bias[r];
                    if (residual) s += residual[r];
                    y[r] = s;
                }
            } else {
                const float v = r < n ? silu_mul(s, s2) : 0.0f;
                outs[tid] = v;
                if (r < n) y[r] = v;
            }
        }
    }
    if constexpr (MODE == 1 && RPB % 16 == 0) {
        // yq needs blocks that own whole 16-groups; the launchers reject it otherwise.
        if (!yq) return;
        __syncthreads();
        if (tid < static_cast<uint32_t>(RPB / 16) && blk_row0 + 16 * tid < n) {
            xgroup_encode_from(outs + 16 * tid, yq + (blk_row0 / 16 + tid));
        }
    }
}

template <uint32_t T, int R, int OPR, int MODE, bool NORM = false, bool ROUTE = false>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                                                   size_t row_bytes, const float* __restrict__ x,
                                                   const XGroup* __restrict__ xq, const float* __restrict__ bias,
                                                   const float* __restrict__ residual, float* __restrict__ y,
                                                   XGroup* __restrict__ yq, uint32_t n, uint32_t units,
                                                   uint32_t kblocks, const Batch batch,
                                                   const float* __restrict__ gamma = nullptr, float eps = 0.0f,
                                                   const MoeCombine cmb = MoeCombine()) {
    gemv_block<T, R, OPR, MODE, NORM, ROUTE>(w, w2, row_bytes, x, xq, bias, residual, y, yq, n, units, kblocks,
                                             batch, gamma, eps, blockIdx.x, blockIdx.y, cmb);
}

struct GemvMulti {
    GemvJob job[kMultiJobs];
    uint32_t jobs;
    uint32_t kblocks;  // k / 32
    const float* x;
    const float* gamma;
    float eps;
    float* norm;
    XGroup* normq;
};

// Grouped launch: up to kMultiJobs GEMVs of one normalised input row (NORM
// prologue), each job with its own weights, type and form, the blocks of job
// p following those of job p - 1. One tiling per (type, form): 2 rows x 8
// octets (MODE 0) and 2 rows x 4 octets (MODE 1, 16-row blocks, so the XGroup
// output is allowed) for quantized weights, 1 row x 32 octets for F32 (MODE
// 0). Block 0 of the launch also stores the normalised row and its XGroup
// form (norm, normq; nullable) for later launches.
// The kernel's registers are the most any compiled-in body needs, and Q6_K
// needs the most (about 100 VGPRs plain, 150 as SwiGLU, against 75-90 for the
// other types), so the Q6_K bodies are compiled in only for launches that
// have such a job (HEAVY: kMultiQ6K, kMultiQ6KSwiGLU). Without the Q6_K
// SwiGLU body the kernel fits 96 VGPRs (5 waves per SIMD) without scratch.
// Forms of a job: 0 = MODE 0 (208; F32 132), 1 = SwiGLU with XGroup output
// (204: 16-row blocks), 2 = SwiGLU without it (108: 4-row blocks, four times
// the blocks).
constexpr int multi_tiling(uint32_t type, int form) {
    return type == kF32 ? 132 : (form == 1 ? 204 : form == 2 ? 108 : 208);
}
constexpr uint32_t kMultiQ6K = 1, kMultiQ6KSwiGLU = 2;

template <uint32_t HEAVY>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HEAVY <= kMultiQ6K ? 5 : 1)))
void gemv_multi_kernel(const GemvMulti m) {
    uint32_t p = 0, bx = blockIdx.x;
    while (p + 1 < m.jobs && bx >= m.job[p].blocks) {
        bx -= m.job[p].blocks;
        ++p;
    }
    const uint32_t k = m.kblocks * 32;
    if (blockIdx.x == 0 && m.norm) {
        rmsnorm_row_lean(m.x, m.gamma, m.norm, m.normq, k, m.eps);
        __syncthreads();  // the prologue below reuses the norm's LDS
    }
    const GemvJob& j = m.job[p];
    const auto* w = static_cast<const uint8_t*>(j.w);
    const auto* w2 = static_cast<const uint8_t*>(j.w2);
    const uint32_t units = (k + Unit<kQ8_0>::elems - 1) / Unit<kQ8_0>::elems;  // 128-value units
    const uint32_t units256 = (k + 255) / 256;
    const Batch b;
#define HIPLLM_MULTI(TT, MM, RR, OO, UU)                                                                            gemv_block<TT, RR, OO, MM, true>(w, w2, j.row_bytes, m.x, nullptr, j.bias, j.residual, j.y, j.yq, j.n, UU,                                      m.kblocks, b, m.gamma, m.eps, bx, 0)
    const uint32_t form = j.mode == 0 ? 0 : (j.yq ? 1 : 2);
    switch (j.type * 3 + form) {
    case kQ4_K * 3: HIPLLM_MULTI(kQ4_K, 0, 2, 8, units256); break;
    case kQ4_K * 3 + 1: HIPLLM_MULTI(kQ4_K, 1, 2, 4, units256); break;
    case kQ4_K * 3 + 2: HIPLLM_MULTI(kQ4_K, 1, 1, 8, units256); break;
    case kQ6_K * 3:
        if constexpr ((HEAVY & kMultiQ6K) != 0) HIPLLM_MULTI(kQ6_K, 0, 2, 8, units256);
        break;
    case kQ6_K * 3 + 1:
        if constexpr ((HEAVY & kMultiQ6KSwiGLU) != 0) HIPLLM_MULTI(kQ6_K, 1, 2, 4, units256);
        break;
    case kQ6_K * 3 + 2:
        if constexpr ((HEAVY & kMultiQ6KSwiGLU) != 0) HIPLLM_MULTI(kQ6_K, 1, 1, 8, units256);
        break;
    case kQ8_0 * 3: HIPLLM_MULTI(kQ8_0, 0, 2, 8, units); break;
    case kQ8_0 * 3 + 1: HIPLLM_MULTI(kQ8_0, 1, 2, 4, units); break;
    case kQ8_0 * 3 + 2: HIPLLM_MULTI(kQ8_0, 1, 1, 8, units); break;
    case kQ5_0 * 3: HIPLLM_MULTI(kQ5_0, 0, 2, 8, units); break;
    case kQ5_0 * 3 + 1: HIPLLM_MULTI(kQ5_0, 1, 2, 4, units); break;
    case kQ5_0 * 3 + 2: HIPLLM_MULTI(kQ5_0, 1, 1, 8, units); break;
    case kF32 * 3: HIPLLM_MULTI(kF32, 0, 1, 32, units256); break;
    default: break;  // rejected by the launcher
    }
#undef HIPLLM_MULTI
}

// XGroup form of x, one thread per 16-group.
__global__ void prep_x_kernel(const float* __restrict__ x, XGroup* __restrict__ xq, uint32_t groups) {
    const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    xgroup_encode_from(x + 16 * static_cast<size_t>(g), xq + g);
}

// Tiling code: 100 * R + OPR.
constexpr int kTilings[] = {108, 116, 132, 202, 204, 208, 216, 232, 401, 402, 404, 408, 416, 432, 802, 804, 808, 816, 832};

// The XGroup output of the SwiGLU form needs blocks that own whole 16-groups
// of it: rows per block (32 / OPR) R must be a multiple of 16.
constexpr bool writes_whole_groups(int t) {
    return (32 / (t % 100)) * (t / 100) % 16 == 0;
}

template <uint32_t T, int MODE>
int launch_typed(int tiling, const void* w, const void* w2, size_t row_bytes, const float* x, const XGroup* xq,
                 const float* bias, const float* residual, float* y, XGroup* yq, uint32_t n, uint32_t units,
                 uint32_t kblocks, hipStream_t stream, const Batch& batch = Batch(), uint32_t vectors = 1) {
    const auto* wp = static_cast<const uint8_t*>(w);
    const auto* wp2 = static_cast<const uint8_t*>(w2);
    const int R = tiling / 100, OPR = tiling % 100;
    if (R < 1 || OPR < 1 || 32 % OPR != 0) return kInvalidArgument;
    const uint32_t rpb = 32u / OPR * R;
    if (MODE == 1 && yq && !writes_whole_groups(tiling)) return kInvalidArgument;
    const dim3 grid((n + rpb - 1) / rpb, vectors);
    switch (tiling) {
#define HIPLLM_GEMV_CASE(RR, OO)                                                                               \
    case 100 * RR + OO:                                                                                        \
        HIPLLM_LAUNCH((gemv_kernel<T, RR, OO, MODE>), grid, dim3(256), 0, stream, wp, wp2, row_bytes,     \
                           x, xq, bias, residual, y, yq, n, units, kblocks, batch);                            \
        break;
        HIPLLM_GEMV_CASE(1, 8)
        HIPLLM_GEMV_CASE(1, 16)
        HIPLLM_GEMV_CASE(1, 32)
        HIPLLM_GEMV_CASE(2, 2)
        HIPLLM_GEMV_CASE(2, 4)
        HIPLLM_GEMV_CASE(2, 8)
        HIPLLM_GEMV_CASE(2, 16)
        HIPLLM_GEMV_CASE(2, 32)
        HIPLLM_GEMV_CASE(4, 1)
        HIPLLM_GEMV_CASE(4, 2)
        HIPLLM_GEMV_CASE(4, 4)
        HIPLLM_GEMV_CASE(4, 8)
        HIPLLM_GEMV_CASE(4, 16)
        HIPLLM_GEMV_CASE(4, 32)
        HIPLLM_GEMV_CASE(8, 2)
        HIPLLM_GEMV_CASE(8, 4)
        HIPLLM_GEMV_CASE(8, 8)
        HIPLLM_GEMV_CASE(8, 16)
        HIPLLM_GEMV_CASE(8, 32)
#undef HIPLLM_GEMV_CASE
    default:
        return kInvalidArgument;
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

// The NORM forms: quantized types, tilings 204 (SwiGLU only), 208, 216, 408, 416.
template <uint32_t T, int MODE>
int launch_typed_norm(int tiling, const void* w, const void* w2, size_t row_bytes, const float* x,
                      const float* gamma, float eps, const float* bias, const float* residual, float* y, XGroup* yq,
                      uint32_t n, uint32_t units, uint32_t kblocks, hipStream_t stream,
                      const MoeCombine& cmb = MoeCombine()) {
    const auto* wp = static_cast<const uint8_t*>(w);
    const auto* wp2 = static_cast<const uint8_t*>(w2);
    if (tiling != 204 && tiling != 208 && tiling != 216 && tiling != 408 && tiling != 416) return kInvalidArgument;
    const uint32_t rpb = 32u / (tiling % 100) * (tiling / 100);
    if (MODE == 1 && yq && !writes_whole_groups(tiling)) return kInvalidArgument;
    const dim3 grid((n + rpb - 1) / rpb);
    const uint32_t lds = kblocks * 32 / 16 * static_cast<uint32_t>(sizeof(XGroup));
    switch (tiling) {
#define HIPLLM_GEMV_NORM_CASE(RR, OO)                                                                         \
    case 100 * RR + OO:                                                                                       \
        HIPLLM_LAUNCH((gemv_kernel<T, RR, OO, MODE, true>), grid, dim3(256), lds, stream, wp, wp2,        \
                           row_bytes, x, nullptr, bias, residual, y, yq, n, units, kblocks, Batch(), gamma,   \
                           eps, cmb);                                                                         \
        break;
        HIPLLM_GEMV_NORM_CASE(2, 4)
        HIPLLM_GEMV_NORM_CASE(2, 8)
        HIPLLM_GEMV_NORM_CASE(2, 16)
        HIPLLM_GEMV_NORM_CASE(4, 8)
        HIPLLM_GEMV_NORM_CASE(4, 16)
#undef HIPLLM_GEMV_NORM_CASE
    default:
        return kInvalidArgument;
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

template <int MODE>
int launch_any_norm(uint32_t type, int tiling, const void* w, const void* w2, size_t row_bytes, const float* x,
                    const float* gamma, float eps, const float* bias, const float* residual, float* y, XGroup* yq,
                    uint32_t n, uint32_t units, uint32_t kblocks, hipStream_t stream,
                    const MoeCombine& cmb = MoeCombine()) {
    switch (type) {
    case kQ4_K: return launch_typed_norm<kQ4_K, MODE>(tiling, w, w2, row_bytes, x, gamma, eps, bias, residual, y, yq, n, units, kblocks, stream, cmb);
    case kQ6_K: return launch_typed_norm<kQ6_K, MODE>(tiling, w, w2, row_bytes, x, gamma, eps, bias, residual, y, yq, n, units, kblocks, stream, cmb);
    case kQ8_0: return launch_typed_norm<kQ8_0, MODE>(tiling, w, w2, row_bytes, x, gamma, eps, bias, residual, y, yq, n, units, kblocks, stream, cmb);
    case kQ5_0: return launch_typed_norm<kQ5_0, MODE>(tiling, w, w2, row_bytes, x, gamma, eps, bias, residual, y, yq, n, units, kblocks, stream, cmb);
    default: return kInvalidArgument;
    }
}

template <int MODE>
int launch_any(uint32_t type, int tiling, const void* w, const void* w2, size_t row_bytes, const float* x,
               const XGroup* xq, const float* bias, const float* residual, float* y, XGroup* yq, uint32_t n,
               uint32_t units, uint32_t kblocks, hipStream_t stream, const Batch& batch = Batch(),
               uint32_t vectors = 1) {
    switch (type) {
    case kQ4_K: return launch_typed<kQ4_K, MODE>(tiling, w, w2, row_bytes, x, xq, bias, residual, y, yq, n, units, kblocks, stream, batch, vectors);
    case kQ6_K: return launch_typed<kQ6_K, MODE>(tiling, w, w2, row_bytes, x, xq, bias, residual, y, yq, n, units, kblocks, stream, batch, vectors);
    case kQ8_0: return launch_typed<kQ8_0, MODE>(tiling, w, w2, row_bytes, x, xq, bias, residual, y, yq, n, units, kblocks, stream, batch, vectors);
    case kQ5_0: return launch_typed<kQ5_0, MODE>(tiling, w, w2, row_bytes, x, xq, bias, residual, y, yq, n, units, kblocks, stream, batch, vectors);
    case kF32: return launch_typed<kF32, MODE>(tiling, w, w2, row_bytes, x, xq, bias, residual, y, yq, n, units, kblocks, stream, batch, vectors);
    case kF16: return launch_typed<kF16, MODE>(tiling, w, w2, row_bytes, x, xq, bias, residual, y, yq, n, units, kblocks, stream, batch, vectors);
    default: return kInvalidArgument;
    }
}

uint32_t unit_elems(uint32_t type) {
    switch (type) {
    case kQ4_K: case kQ6_K: case kF32: case kF16: return 256;
    case kQ8_0: case kQ5_0: return 128;
    default: return 0;
    }
}

bool float_type(uint32_t type) { return type == kF32 || type == kF16; }

bool valid_tiling(int t) {
    for (int v : kTilings) {
        if (v == t) return true;
    }
    return false;
}

// Shared argument checks of the three entry points. k values per row: a
// multiple of 256 for the super-block and float types, of 32 for Q8_0 /
// Q5_0 (a last unit of fewer than 4 blocks is handled in the kernel).
int check_common(uint32_t type, const void* w, const void* w2, size_t row_bytes, const float* x, const XGroup* xq,
                 size_t n, size_t k, size_t expert_stride = 0) {
    const uint32_t ue = unit_elems(type);
    if (!w || n == 0 || k == 0 || ue == 0) return kInvalidArgument;
    const uint32_t be = block_elems(type);
    if (float_type(type) ? k % 256 != 0 : (k % be != 0 || k % 16 != 0)) return kInvalidArgument;
    if (row_bytes < k / be * block_bytes(type)) return kInvalidArgument;
    if (float_type(type) ? !x : !xq) return kInvalidArgument;
    if (x && reinterpret_cast<uintptr_t>(x) % 16 != 0) return kInvalidArgument;
    if (xq && reinterpret_cast<uintptr_t>(xq) % 16 != 0) return kInvalidArgument;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w), ua = reinterpret_cast<uintptr_t>(w2);
    const bool need16 = type == kQ4_K || float_type(type);
    if (need16 && (row_bytes % 16 != 0 || wa % 16 != 0 || ua % 16 != 0 || expert_stride % 16 != 0)) {
        return kInvalidArgument;
    }
    if (wa % 2 != 0 || ua % 2 != 0 || row_bytes % 2 != 0 || expert_stride % 2 != 0) return kInvalidArgument;
    if (n > 0x7fffffffu || k > 0x7fffffffu) return kLengthError;
    return kOk;
}

// Measured choices on MI355X (graph-timed sweeps over the codes at the
// Qwen2.5-7B and Qwen3.5-35B-A3B decode shapes): four rows per octet for tall
// matrices, two for short ones; K split over 16 octets (two waves) once rows
// hold >= 12 units, so each lane streams about one unit and every wave issues
// all its loads at once; 8 rows x 2 octets for LM-head-sized matrices. Tall
// Q4_K matrices of short rows take 8 rows per octet (3584 -> 18944: 12.5 us
// against 13.0 at 4 rows; the grid of 16-row blocks then fits one round of
// resident waves). The SwiGLU form (16-row blocks) measured best at 4 rows x
// 8 octets for FFN widths and 2 x 4 for expert widths. Two units per lane
// per step (all loads of both issued first) measured no faster on the long
// rows (3584 x 18944: 15.0 us against 14.1).
int gemv_pick_shape(uint32_t type, uint32_t n, uint32_t units, int mode) {
    if (type == kF32 || type == kF16 || mode == 1 || n < 1024) return gemv_default_tiling(n, units, mode);
    if (n >= 65536) return 802;
    if (type == kQ4_K && n >= 16384 && units < 32) return 816;
    // Long rows (down projections) amortise the row setup over more units: 4 rows per octet.
    const int R = (n >= 16384 || units >= 32) ? 4 : 2;
    const int OPR = units >= 12 ? 16 : 8;
    return 100 * R + OPR;
}

// ------------------------------------------------- Q4_K and Q6_K on MFMA
//
// The decode GEMV of Q4_K and Q6_K weights held in the x16 tile-packed form,
// with its integer products on the matrix cores (v_mfma_i32_16x16x64_i8).
//
// Packed form: rows in tiles of 16 (a partial last tile is zero-padded);
// tile T, unit (256-value super-block) u takes 16 * B contiguous bytes at
// (T * units + u) * 16 B (B = 144 for Q4_K, 210 for Q6_K): the same bytes as
// the 16 GGUF rows' blocks, ordered so that a wave reads each tile-unit as
// fully contiguous 1 KiB loads (lane l = 16 s + r: row r, k-slice s). In the
// GGUF row order the same wave touches 16 rows kilobytes apart, which
// measured 1.5x slower as a pure read on MI355X.
// * Q4_K (2304 bytes): the 16 rows' 16-byte headers (d, dmin, scales[12]);
//   at 256 + 16 l the quant bytes [16 s, 16 s + 16) of row r; at 1280 + 16 l
//   its bytes [64 + 16 s, 64 + 16 s + 16).
// * Q6_K (3360 bytes), with ql = bytes 0..127, qh = 128..191 of a row's
//   block: at 16 l, ql[64 (s >> 1) + 16 (s & 1), +16); at 1024 + 16 l,
//   ql[64 (s >> 1) + 32 + 16 (s & 1), +16); at 2048 + 16 l,
//   qh[32 (s >> 1) + 16 (s & 1), +16); at 3072 + 16 r the row's 16 scale
//   bytes; at 3328 + 2 r its d.
//
// Product: a wave owns one 16-row tile (the MFMA's N); lane l holds row
// r = l % 16 and k-slice s = l / 16 of each 64-value product, and each MFMA
// sums 16 values of one 16-value activation group per slice.
// * Q4_K: the low nibbles of a lane's first 16 bytes feed MFMA 0, their high
//   nibbles MFMA 1, the second 16 bytes MFMAs 2, 3. Slice s of MFMA i is the
//   group 8 (i >> 1) + 4 (s >> 1) + 2 (i & 1) + (s & 1) of the unit, in
//   sub-block 4 (i >> 1) + 2 (s >> 1) + (i & 1) (model.cpp:616-644 places
//   low nibbles of bytes 32 j .. 32 j + 31 at elements 64 j .., the high
//   nibbles 32 elements later).
// * Q6_K: MFMA i takes quarter i of each 128-value half (model.cpp:646-683:
//   value l + 32 i of half h is ql[64 h + l + 32 (i & 1)]'s nibble i >> 1
//   with bits 2 i, 2 i + 1 of qh[32 h + l] above it); slice s of MFMA i is
//   the group 8 (s >> 1) + 2 i + (s & 1), scaled by scale byte of the same
//   index. The 6-bit quant q enters the MFMA as it is; the -32 is applied
//   with the group's FP32 sum.
// * A's 16 rows are (group slice g, digit d): row 4 g + d holds digit d of
//   the XGroup of slice g at k-slice g and zeros elsewhere (d = 3: zero). C
//   row 4 g + d, column r is then the sum over the group's 16 values of
//   q * digit d, so lane l receives digits 0..2 of its own slice's group for
//   its row. Q4_K combines them exactly in int32, t = c0 + 256 c1 + 65536 c2
//   (|t| <= 16 * 15 * 8355711 < 2^31); Q6_K's 6-bit quants would overflow
//   that, so its three (exact) digit sums are combined in FP32.
// * Each wave stages the 16 XGroups of its current unit in LDS, beside a
//   zero region: the 12 lanes with (l % 16) / 4 == l / 16, (l % 16) % 4 < 3
//   read their A slice from the groups, the others read zeros, with no
//   branch.
// * Each lane adds its groups' scaled sums into one FP32 accumulator; the
//   waves of a block split the units round-robin and are summed in wave
//   order, the four lanes of a row by two xor shuffles: deterministic.
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kMfmaZeroBytes = 784;  // covers the A reads at offsets 0..768 (+16 bytes; Q8_0's last MFMA)

__device__ __forceinline__ i32x4 nibbles(const uint4& q, bool high) {
    i32x4 b;
    if (high) {
        b.x = static_cast<int>((q.x >> 4) & 0x0f0f0f0fu);
        b.y = static_cast<int>((q.y >> 4) & 0x0f0f0f0fu);
        b.z = static_cast<int>((q.z >> 4) & 0x0f0f0f0fu);
        b.w = static_cast<int>((q.w >> 4) & 0x0f0f0f0fu);
    } else {
        b.x = static_cast<int>(q.x & 0x0f0f0f0fu);
        b.y = static_cast<int>(q.y & 0x0f0f0f0fu);
        b.z = static_cast<int>(q.z & 0x0f0f0f0fu);
        b.w = static_cast<int>(q.w & 0x0f0f0f0fu);
    }
    return b;
}

template <uint32_t QT>
struct X16;

template <>
struct X16<kQ4_K> {
    static constexpr uint32_t kBlock = 144;
    struct Unit {
        uint4 hd;      // this lane's row header
        uint4 q0, q1;  // quant bytes 16 s .. and 64 + 16 s ..
    };
    __device__ static Unit load(const uint8_t* tu, uint32_t r, uint32_t, uint32_t lane) {
        Unit v;
        v.hd = ldw128(tu + 16 * r);  // four lanes per header: cached
        v.q0 = ldw128_nt(tu + 256 + 16 * lane);
        v.q1 = ldw128_nt(tu + 1280 + 16 * lane);
        return v;
    }
    // LDS byte offset of slice s's group in MFMA 0 (MFMA i adds group_step(i)).
    __device__ static uint32_t group_base(uint32_t s) { return 64 * (4 * (s >> 1) + (s & 1)); }
    static constexpr uint32_t group_step(int i) { return 512 * (i >> 1) + 128 * (i & 1); }
    // One unit of a lane: four MFMAs, each followed by its group's scaling.
    // a_src: LDS bytes of this lane's A slice for MFMA 0 (the zero region
    // for lanes without A data); se_src: the (sum, e) pair of its slice's
    // group for MFMA 0.
    __device__ static float unit(const Unit& wu, const uint8_t* a_src, const uint8_t* se_src, uint32_t, uint32_t s,
                                 float acc) {
        const uint32_t h0 = wu.hd.x, h1 = wu.hd.y, h2 = wu.hd.z, h3 = wu.hd.w;
        const float d = half_lo(h0), dmin = half_hi(h0);
        // 6-bit scale / min bytes of sub-blocks 0..3 (lo) and 4..7 (hi)
        // (get_scale_min_k4, model.cpp:524-537), shifted to this lane's pair.
        const uint32_t sh = (s >> 1) * 16;
        const uint32_t slo = (h1 & 0x3f3f3f3fu) >> sh, mlo = (h2 & 0x3f3f3f3fu) >> sh;
        const uint32_t shi = ((h3 & 0x0f0f0f0fu) | ((h1 >> 2) & 0x30303030u)) >> sh;
        const uint32_t mhi = (((h3 >> 4) & 0x0f0f0f0fu) | ((h2 >> 2) & 0x30303030u)) >> sh;
        i32x4 a[4];
        float2 se[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = *reinterpret_cast<const i32x4*>(a_src + group_step(i));
            se[i] = *reinterpret_cast<const float2*>(se_src + group_step(i));
        }
        const i32x4 zero = {0, 0, 0, 0};
        float sum_t = 0.0f, sum_m = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = i >> 1, h = i & 1;
            const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], nibbles(p ? wu.q1 : wu.q0, h != 0), zero, 0, 0, 0);
            const int t = c.x + (c.y << 8) + (c.z << 16);
            const uint32_t sc = p ? shi : slo, mn = p ? mhi : mlo;
            const float scale = h ? ubyte1(sc) : ubyte0(sc);
            const float mins = h ? ubyte1(mn) : ubyte0(mn);
            sum_t = fmaf(static_cast<float>(t), se[i].y * scale, sum_t);
            sum_m = fmaf(mins, se[i].x, sum_m);
        }
        return fmaf(d, sum_t, fmaf(-dmin, sum_m, acc));
    }
};

template <>
struct X16<kQ6_K> {
    static constexpr uint32_t kBlock = 210;
    struct Unit {
        uint4 qa, qb, qh;  // ql[64 h + 16 (s & 1) ..], ql[64 h + 32 + ..], qh[32 h + 16 (s & 1) ..]
        uint2 sc;          // scale bytes 8 (s >> 1) .. 8 (s >> 1) + 7 of the row
        uint32_t d;        // the f16 d of rows r & ~1, r | 1
    };
    __device__ static Unit load(const uint8_t* tu, uint32_t r, uint32_t s, uint32_t lane) {
        Unit v;
        v.qa = ldw128_nt(tu + 16 * lane);
        v.qb = ldw128_nt(tu + 1024 + 16 * lane);
        v.qh = ldw128_nt(tu + 2048 + 16 * lane);
        v.sc = *reinterpret_cast<const uint2*>(tu + 3072 + 16 * r + 8 * (s >> 1));
        v.d = ldw32(tu + 3328 + 4 * (r >> 1));
        return v;
    }
    __device__ static uint32_t group_base(uint32_t s) { return 64 * (8 * (s >> 1) + (s & 1)); }
    static constexpr uint32_t group_step(int i) { return 128 * i; }
    // Bytes of MFMA i's B operand: the low (i < 2) or high nibbles of qa / qb
    // (i even / odd) with qh's bits 2 i, 2 i + 1 at bits 4, 5.
    __device__ static uint32_t quant6(uint32_t lo, uint32_t hi, int i) {
        const uint32_t l = (i >> 1) ? (lo >> 4) & 0x0f0f0f0fu : lo & 0x0f0f0f0fu;
        const uint32_t h = i == 0 ? hi << 4 : i == 1 ? hi << 2 : i == 2 ? hi : hi >> 2;
        return (h & 0x30303030u) | l;
    }
    __device__ static float unit(const Unit& wu, const uint8_t* a_src, const uint8_t* se_src, uint32_t r, uint32_t s,
                                 float acc) {
        const float d = (r & 1) ? half_hi(wu.d) : half_lo(wu.d);
        i32x4 a[4];
        float2 se[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = *reinterpret_cast<const i32x4*>(a_src + group_step(i));
            se[i] = *reinterpret_cast<const float2*>(se_src + group_step(i));
        }
        const i32x4 zero = {0, 0, 0, 0};
        const uint32_t sb = 8 * (s & 1);  // this lane's scale byte within each byte pair
        float sum_t = 0.0f, sum_m = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4& lo = (i & 1) ? wu.qb : wu.qa;
            i32x4 b;
            b.x = static_cast<int>(quant6(lo.x, wu.qh.x, i));
            b.y = static_cast<int>(quant6(lo.y, wu.qh.y, i));
            b.z = static_cast<int>(quant6(lo.z, wu.qh.z, i));
            b.w = static_cast<int>(quant6(lo.w, wu.qh.w, i));
            const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b, zero, 0, 0, 0);
            const float t = fmaf(65536.0f, static_cast<float>(c.z),
                                 fmaf(256.0f, static_cast<float>(c.y), static_cast<float>(c.x)));
            // Scale byte (s & 1) + 2 i of this lane's eight (signed).
            const uint32_t word = (i >> 1) ? wu.sc.y : wu.sc.x;
            const float scale = static_cast<float>(static_cast<int8_t>(word >> (sb + 16 * (i & 1))));
            sum_t = fmaf(t, se[i].y * scale, sum_t);
            sum_m = fmaf(scale, se[i].x, sum_m);
        }
        return fmaf(d, fmaf(-32.0f, sum_m, sum_t), acc);
    }
};

// Q8_0 (34-byte blocks of 32 values: f16 d, 32 int8 quants): a tile-unit
// holds for MFMA i and lane l = 16 s + r the 16 quants of row r at values
// [64 i + 16 s, +16) of the unit (block 2 i + (s >> 1), bytes 16 (s & 1)
// on), 1 KiB per MFMA, then per row its eight d values ordered so that a
// lane reads the four of its blocks 2 i + (s >> 1) as one 8-byte word. The
// quants are the MFMA's B operand as they are (signed bytes); MFMA i's A
// slices are groups 4 i .. 4 i + 3 of the unit, so each lane's result is one
// group's three exact digit sums for its row, combined in FP32 (their
// magnitude can exceed int32) and scaled by the group's e and the block's d.
template <>
struct X16<kQ8_0> {
    static constexpr uint32_t kBlock = 272;  // 8 blocks of 34 bytes per row and unit
    struct Unit {
        uint4 q[4];  // MFMA i's quant slice
        uint2 d;     // this lane's four block scales (f16), MFMA 0..3
    };
    __device__ static Unit load(const uint8_t* tu, uint32_t r, uint32_t s, uint32_t lane) {
        Unit v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v.q[i] = ldw128_nt(tu + 1024 * i + 16 * lane);
        v.d = *reinterpret_cast<const uint2*>(tu + 4096 + 16 * r + 8 * (s >> 1));
        return v;
    }
    __device__ static uint32_t group_base(uint32_t s) { return 64 * s; }
    static constexpr uint32_t group_step(int i) { return 256 * i; }
    __device__ static float unit(const Unit& wu, const uint8_t* a_src, const uint8_t* se_src, uint32_t, uint32_t,
                                 float acc) {
        i32x4 a[4];
        float2 se[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = *reinterpret_cast<const i32x4*>(a_src + group_step(i));
            se[i] = *reinterpret_cast<const float2*>(se_src + group_step(i));
        }
        const i32x4 zero = {0, 0, 0, 0};
        const float dv[4] = {half_lo(wu.d.x), half_hi(wu.d.x), half_lo(wu.d.y), half_hi(wu.d.y)};
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            i32x4 b;
            b.x = static_cast<int>(wu.q[i].x);
            b.y = static_cast<int>(wu.q[i].y);
            b.z = static_cast<int>(wu.q[i].z);
            b.w = static_cast<int>(wu.q[i].w);
            const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b, zero, 0, 0, 0);
            const float t = fmaf(65536.0f, static_cast<float>(c.z),
                                 fmaf(256.0f, static_cast<float>(c.y), static_cast<float>(c.x)));
            sum = fmaf(t, se[i].y * dv[i], sum);
        }
        return acc + sum;
    }
};

// y = W x (+ bias) (+ residual) for x16-packed W of type QT. A block of WPB
// waves owns RT consecutive 16-row tiles; its waves split the units
// round-robin and each wave multiplies every unit it takes into all RT
// tiles, so one copy of the unit's activation groups serves 16 RT rows. Per
// unit a lane loads 16 bytes of x's XGroups (the unit's 16 groups are 1 KiB,
// one load per lane) with the unit's weights; the wave stores them to its
// own 1 KiB of LDS and reads its A slices and (sum, e) pairs from there. Each
// wave also keeps a zero region that the lanes without A data read instead.
// No block barrier before the products: a wave starts as soon as its first
// unit has landed.
// MODE 0: y = W x (+ bias) (+ residual). MODE 1 (the FFN gate/up of one
// row): w2 is the up matrix in the same form, y = silu(W x) * (W2 x) (the
// reference's SwiGLU, cpu_llm.cpp:188-202) and yq (nullable) receives the
// XGroup form of y, one group per 16-row tile (the down projection's input).
// NORM 1 (an RMSNorm before the product): xq holds the XGroup form of
// x * gamma for the raw row x, nrm.sumsq_in its per-16-value sums of squares
// (k / 16 doubles, as a NORM 2 launch writes them); the block reduces them in
// a fixed order (wave 0, lanes strided, then the wave sum) to inv = 1 /
// sqrt(mean + eps) and scales the products by it: W (x * inv * gamma). NORM 2
// (MODE 0; an RMSNorm after y, n % 16 == 0): each 16-row tile of y also
// writes the XGroup form of y * nrm.gamma_out and the double sum of squares
// of its 16 values (in row order), the input of a NORM 1 launch.
//
// RTE (one token's routed expert vectors, grid.y = route j): the weights of
// route j are expert e's rows, e * expert_bytes into the packed copy of the
// whole [experts * n, k] block (n, the rows of one expert, a multiple of
// 16); its input is row j of x (x_routed) or row 0, its output row j of y
// and yq (ldy values apart). RTE 1 reads e = ids[j] (clamped to experts -
// 1); RTE 2 picks the routes itself: the first wave runs the router's
// softmax / top-k / renormalisation (router.h) on the token's logits, and
// block (0, 0) stores the ids and weights for the launches that follow.
struct X16Route {
    const int32_t* ids;
    const float* logits;
    int32_t* ids_out;
    float* weights_out;
    uint32_t experts;
    uint32_t routes;
    size_t expert_bytes;
    uint32_t x_routed;
    uint32_t ldx;
    uint32_t ldy;
};

// CONV (MODE 0 with NORM 3; cv.w nullable): y is the projection of a
// causal conv's input channels (row = channel): each row's value x is
// convolved with its ksize (<= 4) taps over the channel's history rows and
// x, y = conv * sigmoid(conv) (the conv + SiLU of conv1d_silu_kernel), and
// the channel's history shifts by one row with x appended. The tile's taps
// and history are loaded at kernel start.
struct X16Conv {
    const float* w;      // [channels, ksize]
    float* history;      // [ksize - 1, channels]
    uint32_t channels;   // the history's row length (>= n)
    uint32_t ksize;
};
constexpr uint32_t kX16ConvMax = 4;

// The work of block (bx, by); the kernels below call it with their block
// index (or, for a paired launch, the index within the job).
template <uint32_t QT, int WPB, int RT, int MODE, int NORM, int RTE, bool CONV>
__device__ __forceinline__ void x16_body(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                                         const XGroup* __restrict__ xq, const float* __restrict__ bias,
                                         const float* __restrict__ residual, float* __restrict__ y,
                                         XGroup* __restrict__ yq, uint32_t n, uint32_t units, const X16Norm nrm,
                                         const X16Route route, const X16Conv cv, uint32_t bx, uint32_t by) {
    static_assert(NORM != 2 || MODE == 0, "the output norm data comes from plain GEMVs");
    static_assert(RTE == 0 || NORM == 0, "routed vectors take no norm");
    static_assert(NORM != 3 || (MODE == 0 && RT == 1), "the in-block norm serves plain one-tile GEMVs");
    static_assert(!CONV || NORM == 1 || NORM == 3, "the conv epilogue serves the paired launch");
    if constexpr (RTE != 0) {
        const uint32_t j = by;
        uint32_t e;
        if constexpr (RTE == 2) {
            __shared__ int32_t route_id[8];
            __shared__ float route_w[8];
            if (threadIdx.x < 64) {
                topk_row<kRouteMaxExperts / 64>(route.logits, route.experts, route.routes, route_id, route_w,
                                                threadIdx.x);
            }
            __syncthreads();
            if (bx == 0 && j == 0 && threadIdx.x < route.routes) {
                route.ids_out[threadIdx.x] = route_id[threadIdx.x];
                route.weights_out[threadIdx.x] = route_w[threadIdx.x];
            }
            e = min(static_cast<uint32_t>(route_id[j]), route.experts - 1);
        } else {
            e = min(static_cast<uint32_t>(route.ids[j]), route.experts - 1);
        }
        w += static_cast<size_t>(e) * route.expert_bytes;
        if (MODE == 1) w2 += static_cast<size_t>(e) * route.expert_bytes;
        xq += static_cast<size_t>(route.x_routed ? j : 0) * (route.ldx / 16);
        y += static_cast<size_t>(j) * route.ldy;
        if (yq) yq += static_cast<size_t>(j) * (route.ldy / 16);
    }
    using F = X16<QT>;
    constexpr uint32_t kTileUnit = 16 * F::kBlock;
    constexpr int NM = MODE == 1 ? 2 : 1;  // matrices
    constexpr int NA = NM * RT;            // accumulators
    __shared__ __align__(16) uint8_t xs[WPB][2048];
    __shared__ __align__(16) float part[WPB][16 * NA];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t r = lane & 15, s = lane >> 4;
    const uint32_t tiles = (n + 15) / 16;
    const uint32_t tile0 = bx * RT;
    const size_t tile_bytes = static_cast<size_t>(units) * kTileUnit;
    const uint8_t* wt[NA];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        wt[t] = w + min(tile0 + t, tiles - 1) * tile_bytes;
        if (MODE == 1) wt[RT + t] = w2 + min(tile0 + t, tiles - 1) * tile_bytes;
    }
    const uint4* xsrc = reinterpret_cast<const uint4*>(xq);
    // This wave's units: wave, wave + WPB, ... (wave-uniform, kept scalar),
    // counted from a start that rotates with the block: every wave of every
    // block would otherwise read the same unit's activation groups at the
    // same moment, from the same few L2 channels.
    const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t mine = units > wv ? (units - wv + WPB - 1) / WPB : 0;
    const uint32_t rot = bx % units;
    struct Slot {
        uint4 x;
        typename F::Unit w[NA];
    };
    Slot sl;
    auto fill = [&](uint32_t idx) {
        uint32_t u = wv + idx * WPB + rot;
        if (u >= units) u -= units;
        if constexpr (NORM != 3) sl.x = xsrc[64 * u + lane];
#pragma unroll
        for (int t = 0; t < NA; ++t) sl.w[t] = F::load(wt[t] + static_cast<size_t>(u) * kTileUnit, r, s, lane);
    };
    uint8_t* lds = xs[wave];
    if (lane < kMfmaZeroBytes / 16) *reinterpret_cast<uint4*>(lds + 1024 + 16 * lane) = make_uint4(0, 0, 0, 0);
    const bool a_lane = (r >> 2) == s && (r & 3) < 3;
    const uint32_t slot = F::group_base(s);
    const uint8_t* a_src = a_lane ? lds + slot + 16 * (r & 3) : lds + 1024;
    const uint8_t* se_src = lds + slot + 48;
    float acc[NA];
#pragma unroll
    for (int t = 0; t < NA; ++t) acc[t] = 0.0f;
    // One unit in flight per wave, refilled as soon as the unit's bytes have
    // been consumed; the waves of a block, and the blocks of a CU, keep the
    // memory system busy. (With two units in flight the refill of the second
    // sits under a branch that the last pass skips, and the compiler's waits
    // then cover every load in flight.)
    if (mine > 0) fill(0);
    // The epilogue's per-row operands, loaded now rather than after the
    // block reduction (same values, same sums).
    float pre_b = 0.0f, pre_r = 0.0f, pre_g = 0.0f;
    float ctap[kX16ConvMax], chist[kX16ConvMax - 1];
    if (MODE == 0 && tid < 16 * RT) {
        const uint32_t row = tile0 * 16 + tid;
        if (row < n) {
            if (bias) pre_b = bias[row];
            if (residual) pre_r = residual[row];
            if (NORM == 2) pre_g = nrm.gamma_out[row];
            if (CONV && cv.w) {
#pragma unroll
                for (uint32_t j = 0; j < kX16ConvMax; ++j) {
                    ctap[j] = j < cv.ksize ? cv.w[static_cast<size_t>(row) * cv.ksize + j] : 0.0f;
                    if (j + 1 < kX16ConvMax) {
                        chist[j] = j + 1 < cv.ksize ? cv.history[static_cast<size_t>(j) * cv.channels + row] : 0.0f;
                    }
                }
            }
        }
    }
    __shared__ float inv_s;
    if (NORM == 1 && wave == 0) {
        // Up to 512 partials (k <= 8192), all loads issued before the sum.
        const uint32_t tiles_in = 16 * units;
        double v[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t i = lane + 64 * t;
            v[t] = i < tiles_in ? nrm.sumsq_in[i] : 0.0;
        }
        double ss = v[0];
#pragma unroll
        for (int t = 1; t < 8; ++t) ss += v[t];
        ss = wave_sum_d(ss);
        if (lane == 0) {
            const float ms = static_cast<float>(ss / static_cast<double>(256 * units));
            inv_s = 1.0f / sqrtf(ms + nrm.eps);
        }
    }
    // NORM 3: the block normalises the raw input row into LDS (the XGroup
    // form of x * inv * gamma, the same bits as the standalone RMSNorm) while
    // its first weight loads are in flight; the waves read their A slices
    // and (sum, e) pairs straight from there.
    extern __shared__ __align__(16) uint8_t x16_norm_lds[];  // 4 k bytes, sized at launch
    if constexpr (NORM == 3) {
        rmsnorm_row_lean(nrm.x_in, nrm.gamma_in, nullptr, reinterpret_cast<XGroup*>(x16_norm_lds), 256 * units,
                         nrm.eps);
        __syncthreads();
        for (uint32_t idx = 0; idx < mine; ++idx) {
            uint32_t u = wv + idx * WPB + rot;
            if (u >= units) u -= units;
            const uint8_t* xu = x16_norm_lds + 1024 * u;
            const uint8_t* a_u = a_lane ? xu + slot + 16 * (r & 3) : lds + 1024;
#pragma unroll
            for (int t = 0; t < NA; ++t) acc[t] = F::unit(sl.w[t], a_u, xu + slot + 48, r, s, acc[t]);
            if (idx + 1 < mine) fill(idx + 1);
        }
    }
    for (uint32_t idx = 0; NORM != 3 && idx < mine; ++idx) {
        *reinterpret_cast<uint4*>(lds + 16 * lane) = sl.x;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int t = 0; t < NA; ++t) acc[t] = F::unit(sl.w[t], a_src, se_src, r, s, acc[t]);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (idx + 1 < mine) fill(idx + 1);
    }
    // Rows: lanes r, r + 16, r + 32, r + 48 hold the four group slices.
#pragma unroll
    for (int t = 0; t < NA; ++t) {
        float v = acc[t];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (lane < 16) part[wave][16 * t + lane] = v;
    }
    __syncthreads();
    if (tid < 16 * RT) {
        const uint32_t row = tile0 * 16 + tid;
        float v = part[0][tid];
#pragma unroll
        for (int i = 1; i < WPB; ++i) v += part[i][tid];
        if (NORM == 1) v *= inv_s;
        if (MODE == 1) {
            float u = part[0][16 * RT + tid];
#pragma unroll
            for (int i = 1; i < WPB; ++i) u += part[i][16 * RT + tid];
            if (NORM == 1) u *= inv_s;
            v = row < n ? silu_mul(v, u) : 0.0f;
            part[0][tid] = v;  // the tile's outputs, for the XGroup encoding below
        } else if (row < n) {
            if (bias) v += pre_b;
            if (residual) v += pre_r;
            if (CONV && cv.w) {
                // conv1d_silu_kernel's sum: the history rows in order, then x.
                const uint32_t hr = cv.ksize - 1;
                float cacc = 0.0f;
#pragma unroll
                for (uint32_t j = 0; j < kX16ConvMax; ++j) {
                    const float win = j < hr ? chist[j] : v;
                    if (j < cv.ksize) cacc += win * ctap[j];
                    if (j < hr) {
                        const float next = j + 1 < hr ? chist[j + 1 < kX16ConvMax - 1 ? j + 1 : 0] : v;
                        cv.history[static_cast<size_t>(j) * cv.channels + row] = next;
                    }
                }
                v = cacc * sigmoid_ref(cacc);
            }
        }
        if (row < n) y[row] = v;
        if (NORM == 2) {
            // Each thread rewrites only its own slots, after reading them.
            part[0][tid] = row < n ? v * pre_g : 0.0f;
            part[1][tid] = row < n ? v : 0.0f;
        }
    }
    if (MODE == 1 && yq) {
        __syncthreads();
        if (tid < static_cast<uint32_t>(RT) && (tile0 + tid) * 16 < n) xgroup_encode_from(&part[0][16 * tid], yq + tile0 + tid);
    }
    if (NORM == 2) {
        __syncthreads();
        if (tid < static_cast<uint32_t>(RT) && (tile0 + tid) * 16 < n) {
            xgroup_encode_from(&part[0][16 * tid], nrm.yq_out + tile0 + tid);
            double ss = 0.0;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const double t = part[1][16 * tid + i];
                ss += t * t;
            }
            nrm.sumsq_out[tile0 + tid] = ss;
        }
    }
}

template <uint32_t QT, int WPB, int RT, int MODE, int NORM, int RTE = 0>
__global__ __launch_bounds__(64 * WPB) void gemv_x16_kernel(const uint8_t* __restrict__ w,
                                                            const uint8_t* __restrict__ w2,
                                                            const XGroup* __restrict__ xq,
                                                            const float* __restrict__ bias,
                                                            const float* __restrict__ residual,
                                                            float* __restrict__ y, XGroup* __restrict__ yq,
                                                            uint32_t n, uint32_t units, X16Norm nrm,
                                                            X16Route route = X16Route{}) {
    x16_body<QT, WPB, RT, MODE, NORM, RTE, false>(w, w2, xq, bias, residual, y, yq, n, units, nrm, route, X16Conv{},
                                                  blockIdx.x, blockIdx.y);
}

// Two plain GEMVs of one normalised row in one launch (NORM 3: every block
// normalises the raw row itself): blocks [0, blocks_a) compute job A's 16-row
// tiles (with the conv epilogue when cv.w is set), the rest job B's. QA and
// QB are the jobs' x16 types.
struct X16Job {
    const uint8_t* w;
    float* y;
    uint32_t n;
};

// NORM 3: each block normalises the raw row (nrm.x_in, nrm.gamma_in); NORM 1:
// the producer left the XGroup form of x * gamma in xq and the per-16 sums
// of squares in nrm.sumsq_in.
template <uint32_t QA, uint32_t QB, int WPB, int NORM>
__global__ __launch_bounds__(64 * WPB) void gemv_x16_pair_kernel(const X16Job a, const X16Job b, uint32_t blocks_a,
                                                                 uint32_t units, const XGroup* __restrict__ xq,
                                                                 X16Norm nrm, X16Conv cv) {
    if (blockIdx.x < blocks_a) {
        x16_body<QA, WPB, 1, 0, NORM, 0, true>(a.w, nullptr, xq, nullptr, nullptr, a.y, nullptr, a.n, units, nrm,
                                               X16Route{}, cv, blockIdx.x, 0);
    } else {
        x16_body<QB, WPB, 1, 0, NORM, 0, false>(b.w, nullptr, xq, nullptr, nullptr, b.y, nullptr, b.n, units, nrm,
                                                X16Route{}, X16Conv{}, blockIdx.x - blocks_a, 0);
    }
}

// Repacking into the x16 form: one thread per 16-byte chunk of the packed
// bytes; rows past n give zeros. Q4_K (144 chunks per tile-unit: 16
// headers, 64 first slices, 64 second slices) reads 16-byte-aligned rows;
// Q6_K (210 chunks: 64 each of ql / ql / qh slices, 16 scale rows, two
// chunks of eight d values) reads 2-byte-aligned rows in 16-bit pieces.
__device__ __forceinline__ uint4 ld128_a2(const uint8_t* p) {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
    return make_uint4(q[0] | (static_cast<uint32_t>(q[1]) << 16), q[2] | (static_cast<uint32_t>(q[3]) << 16),
                      q[4] | (static_cast<uint32_t>(q[5]) << 16), q[6] | (static_cast<uint32_t>(q[7]) << 16));
}

template <uint32_t QT>
__global__ __launch_bounds__(256) void pack_x16_kernel(const uint8_t* __restrict__ w, size_t row_bytes,
                                                       uint8_t* __restrict__ out, uint32_t n, uint32_t units,
                                                       size_t chunks) {
    constexpr uint32_t B = X16<QT>::kBlock;
    const size_t c = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (c >= chunks) return;
    const size_t tu = c / B;
    const uint32_t j = static_cast<uint32_t>(c % B);
    const uint32_t tile = static_cast<uint32_t>(tu / units), u = static_cast<uint32_t>(tu % units);
    const uint8_t* unit0 = w + static_cast<size_t>(u) * B;  // + row * row_bytes
    uint4 v = make_uint4(0, 0, 0, 0);
    if (QT == kQ4_K) {
        uint32_t r, src;
        if (j < 16) {
            r = j;
            src = 0;
        } else {
            const uint32_t l = (j - 16) % 64;
            r = l & 15;
            src = 16 + 64 * ((j - 16) / 64) + 16 * (l >> 4);
        }
        const uint32_t row = tile * 16 + r;
        if (row < n) v = ldw128(unit0 + static_cast<size_t>(row) * row_bytes + src);
    } else if (QT == kQ8_0) {
        if (j < 256) {
            // MFMA i = j / 64, lane 16 s + r: block 2 i + (s >> 1), quant bytes 16 (s & 1) on.
            const uint32_t i = j / 64, l = j % 64, r = l & 15, s = l >> 4;
            const uint32_t row = tile * 16 + r;
            const uint32_t src = 34 * (2 * i + (s >> 1)) + 2 + 16 * (s & 1);
            if (row < n) v = ld128_a2(unit0 + static_cast<size_t>(row) * row_bytes + src);
        } else {
            // Row j - 256's d values, half 4 p + i = block 2 i + p.
            const uint32_t row = tile * 16 + (j - 256);
            uint32_t hv[8];
#pragma unroll
            for (uint32_t h = 0; h < 8; ++h) {
                const uint32_t blk = 2 * (h & 3) + (h >> 2);
                hv[h] = row < n ? *reinterpret_cast<const uint16_t*>(unit0 + static_cast<size_t>(row) * row_bytes + 34 * blk)
                                : 0u;
            }
            v = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
        }
    } else if (j < 192) {
        const uint32_t part = j / 64, l = j % 64, r = l & 15, s = l >> 4;
        const uint32_t src = part == 2 ? 128 + 32 * (s >> 1) + 16 * (s & 1) : 64 * (s >> 1) + 32 * part + 16 * (s & 1);
        const uint32_t row = tile * 16 + r;
        if (row < n) v = ld128_a2(unit0 + static_cast<size_t>(row) * row_bytes + src);
    } else if (j < 208) {
        const uint32_t row = tile * 16 + (j - 192);
        if (row < n) v = ld128_a2(unit0 + static_cast<size_t>(row) * row_bytes + 192);
    } else {
        uint32_t hv[8];
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            const uint32_t row = tile * 16 + 8 * (j - 208) + i;
            hv[i] = row < n ? *reinterpret_cast<const uint16_t*>(unit0 + static_cast<size_t>(row) * row_bytes + 208) : 0u;
        }
        v = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
    }
    *reinterpret_cast<uint4*>(out + c * 16) = v;
}

// Launch shape code 1000 RT + 100 + WPB (one unit in flight per wave).
// Picked from measurements on MI355X over 16+ rotated weight copies
// (Qwen2.5-7B and -14B shapes). What decides is how many waves are resident
// at once and how evenly the blocks fill the 256 CUs: tall matrices of short
// rows (>= 800 tiles: 3584 -> 18944, 5120 -> 13824) run best with 4 waves per
// block, all resident in one round, and the SwiGLU pair there with two tiles
// per block; long rows (>= 32 units) with 16 waves per block while the tiles
// fit one block per CU (18944 -> 3584), else two tiles per 8-wave block
// (13824 -> 5120); everything else with 8 waves per block.
int x16_default_waves(uint32_t n, uint32_t units, int mode) {
    const uint32_t tiles = (n + 15) / 16;
    if (units >= 32) return tiles <= 256 ? 1116 : 2108;
    if (tiles >= 800) return mode == 1 ? 2104 : 1104;
    return 1108;
}

}  // namespace

// Default tiling from a simple cost model (used for F32 / F16 weights and
// batched launches): the busiest lane's sequential units plus the data per
// resident wave, where fewer than ~1500 waves leave HBM under-fed, and a
// small charge per excess wave and for cross-wave reductions. The SwiGLU form
// takes the measured 16-row-block choice when it writes the XGroup form of
// its output (blocks must own whole 16-groups), the cost model otherwise.
int gemv_default_tiling(uint32_t n, uint32_t units, int mode, uint32_t vectors, bool whole_groups) {
    if (mode == 1 && whole_groups) return n >= 8192 ? 408 : 204;
    int best = 0;
    double best_cost = 0.0;
    for (int t : kTilings) {
        const int R = t / 100, OPR = t % 100;
        const uint32_t rpb = 32u / OPR * R;
        const double blocks = static_cast<double>((n + rpb - 1) / rpb);
        const double waves = blocks * 4.0 * vectors;
        const double per = static_cast<double>((units + OPR - 1) / OPR);  // units of the busiest octet
        const double work = static_cast<double>(n) * units * vectors;
        const double cost = work / (waves < 1536.0 ? waves : 1536.0) + 2.0 * per + 0.5 * waves / 4096.0 +
                            (OPR > 8 ? 0.5 : 0.0);
        if (best == 0 || cost < best_cost) {
            best_cost = cost;
            best = t;
        }
    }
    return best;
}

int launch_prep_x(const float* x, XGroup* xq, size_t k, hipStream_t stream) {
    if (!x || !xq || k == 0 || k % 16 != 0) return kInvalidArgument;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(xq) % 16 != 0) {
        return kInvalidArgument;
    }
    if (k / 16 > 0xffffffffull) return kLengthError;
    const uint32_t groups = static_cast<uint32_t>(k / 16);
    HIPLLM_LAUNCH(prep_x_kernel, dim3((groups + 255) / 256), dim3(256), 0, stream, x, xq, groups);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

namespace {
bool x16_type(uint32_t type) { return type == kQ4_K || type == kQ6_K || type == kQ8_0; }
uint32_t x16_block(uint32_t type) { return type == kQ4_K ? 144u : type == kQ6_K ? 210u : 272u; }
}  // namespace

size_t x16_bytes(uint32_t type, size_t n, size_t k) {
    if (!x16_type(type) || n == 0 || k == 0 || k % 256 != 0) return 0;
    return (n + 15) / 16 * 16 * (k / 256) * x16_block(type);
}

int launch_pack_x16(uint32_t type, const void* w, size_t row_bytes, size_t n, size_t k, void* packed,
                    hipStream_t stream) {
    if (!x16_type(type) || !w || !packed || n == 0 || k == 0 || k % 256 != 0) return kInvalidArgument;
    const uint32_t B = x16_block(type);
    if (row_bytes < k / 256 * B || reinterpret_cast<uintptr_t>(packed) % 16 != 0) return kInvalidArgument;
    // Q4_K rows are read in 16-byte pieces, Q6_K and Q8_0 rows in 16-bit pieces.
    const size_t align = type == kQ4_K ? 16 : 2;
    if (row_bytes % align != 0 || reinterpret_cast<uintptr_t>(w) % align != 0) return kInvalidArgument;
    if (n > 0x7fffffffull || k > 0x7fffffffull) return kLengthError;
    const uint32_t units = static_cast<uint32_t>(k / 256);
    const size_t chunks = (n + 15) / 16 * units * B;
    if ((chunks + 255) / 256 > 0x7fffffffull) return kLengthError;
    const dim3 grid(static_cast<uint32_t>((chunks + 255) / 256));
    const auto* wb = static_cast<const uint8_t*>(w);
    auto* out = static_cast<uint8_t*>(packed);
    if (type == kQ4_K) {
        HIPLLM_LAUNCH(pack_x16_kernel<kQ4_K>, grid, dim3(256), 0, stream, wb, row_bytes, out, static_cast<uint32_t>(n),
                      units, chunks);
    } else if (type == kQ8_0) {
        HIPLLM_LAUNCH(pack_x16_kernel<kQ8_0>, grid, dim3(256), 0, stream, wb, row_bytes, out, static_cast<uint32_t>(n),
                      units, chunks);
    } else {
        HIPLLM_LAUNCH(pack_x16_kernel<kQ6_K>, grid, dim3(256), 0, stream, wb, row_bytes, out, static_cast<uint32_t>(n),
                      units, chunks);
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

namespace {
template <uint32_t QT, int MODE, int NORM>
int launch_x16(int code, const uint8_t* wp, const uint8_t* wp2, const XGroup* xq, const float* bias,
               const float* residual, float* y, XGroup* yq, uint32_t nn, uint32_t units, const X16Norm& nrm,
               hipStream_t stream) {
    const uint32_t tiles = (nn + 15) / 16;
    switch (code) {
#define HIPLLM_X16_CASE(RT, W)                                                                                      \
    case 1000 * RT + 100 + W:                                                                                       \
        HIPLLM_LAUNCH((gemv_x16_kernel<QT, W, RT, MODE, NORM>), dim3((tiles + RT - 1) / RT), dim3(64 * W), 0, stream, \
                      wp, wp2, xq, bias, residual, y, yq, nn, units, nrm);                                           \
        break;
        HIPLLM_X16_CASE(1, 4)
        HIPLLM_X16_CASE(1, 8)
        HIPLLM_X16_CASE(1, 16)
        HIPLLM_X16_CASE(2, 4)
        HIPLLM_X16_CASE(2, 8)
        HIPLLM_X16_CASE(2, 16)
#undef HIPLLM_X16_CASE
    default:
        return kInvalidArgument;
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

int check_x16(uint32_t type, const void* packed, const XGroup* xq, const float* y, size_t n, size_t k) {
    if (!x16_type(type) || !packed || !xq || !y || n == 0 || k == 0 || k % 256 != 0) return kInvalidArgument;
    if (reinterpret_cast<uintptr_t>(packed) % 16 != 0 || reinterpret_cast<uintptr_t>(xq) % 16 != 0) {
        return kInvalidArgument;
    }
    if (n > 0x7fffffffull || k > 0x7fffffffull) return kLengthError;
    return kOk;
}
}  // namespace

namespace {
// norm: nullptr or neither input nor output form -> 0; sumsq_in -> 1 (k <= 8192);
// gamma_out -> 2 (plain GEMV, n % 16 == 0, yq_out 16-byte aligned, sumsq_out);
// -1 when the combination is not offered.
int x16_norm_kind(const X16Norm* norm, int mode, size_t n, size_t k) {
    if (!norm || (!norm->sumsq_in && !norm->gamma_out)) return 0;
    if (norm->sumsq_in && norm->gamma_out) return -1;
    if (norm->sumsq_in) return k <= 8192 ? 1 : -1;
    if (mode != 0 || n % 16 != 0 || !norm->yq_out || !norm->sumsq_out) return -1;
    if (reinterpret_cast<uintptr_t>(norm->yq_out) % 16 != 0) return -1;
    return 2;
}

template <uint32_t QT, int MODE>
int launch_x16_norm(int kind, int code, const uint8_t* wp, const uint8_t* wp2, const XGroup* xq, const float* bias,
                    const float* residual, float* y, XGroup* yq, uint32_t nn, uint32_t units, const X16Norm* norm,
                    hipStream_t stream) {
    const X16Norm nrm = norm ? *norm : X16Norm{};
    if (kind == 1) return launch_x16<QT, MODE, 1>(code, wp, wp2, xq, bias, residual, y, yq, nn, units, nrm, stream);
    if constexpr (MODE == 0) {
        if (kind == 2) return launch_x16<QT, 0, 2>(code, wp, wp2, xq, bias, residual, y, yq, nn, units, nrm, stream);
    }
    return launch_x16<QT, MODE, 0>(code, wp, wp2, xq, bias, residual, y, yq, nn, units, nrm, stream);
}
}  // namespace

int launch_gemv_x16(uint32_t type, const void* packed, const XGroup* xq, const float* bias, const float* residual,
                    float* y, size_t n, size_t k, int waves, hipStream_t stream, const X16Norm* norm) {
    const int rc = check_x16(type, packed, xq, y, n, k);
    if (rc != kOk) return rc;
    const int kind = x16_norm_kind(norm, 0, n, k);
    if (kind < 0) return kInvalidArgument;
    const uint32_t units = static_cast<uint32_t>(k / 256), nn = static_cast<uint32_t>(n);
    const int code = waves ? waves : x16_default_waves(nn, units, 0);
    const auto* wp = static_cast<const uint8_t*>(packed);
    if (type == kQ8_0) {
        // Q8_0 copies serve plain products (no norm data in or out).
        if (kind != 0) return kInvalidArgument;
        return launch_x16<kQ8_0, 0, 0>(code, wp, nullptr, xq, bias, residual, y, nullptr, nn, units, X16Norm{},
                                       stream);
    }
    return type == kQ4_K
               ? launch_x16_norm<kQ4_K, 0>(kind, code, wp, nullptr, xq, bias, residual, y, nullptr, nn, units, norm,
                                           stream)
               : launch_x16_norm<kQ6_K, 0>(kind, code, wp, nullptr, xq, bias, residual, y, nullptr, nn, units, norm,
                                           stream);
}

int launch_gemv_x16_swiglu(uint32_t type, const void* gate, const void* up, const XGroup* xq, float* y, XGroup* yq,
                           size_t n, size_t k, int waves, hipStream_t stream, const X16Norm* norm) {
    if (type == kQ8_0) return kInvalidArgument;  // Q4_K / Q6_K pairs
    int rc = check_x16(type, gate, xq, y, n, k);
    if (rc == kOk) rc = check_x16(type, up, xq, y, n, k);
    if (rc != kOk) return rc;
    if (yq && (n % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0)) return kInvalidArgument;
    const int kind = x16_norm_kind(norm, 1, n, k);
    if (kind < 0) return kInvalidArgument;
    const uint32_t units = static_cast<uint32_t>(k / 256), nn = static_cast<uint32_t>(n);
    const int code = waves ? waves : x16_default_waves(nn, units, 1);
    const auto* g = static_cast<const uint8_t*>(gate);
    const auto* u = static_cast<const uint8_t*>(up);
    return type == kQ4_K
               ? launch_x16_norm<kQ4_K, 1>(kind, code, g, u, xq, nullptr, nullptr, y, yq, nn, units, norm, stream)
               : launch_x16_norm<kQ6_K, 1>(kind, code, g, u, xq, nullptr, nullptr, y, yq, nn, units, norm, stream);
}

namespace {
template <uint32_t QA, uint32_t QB>
int launch_x16_pair_types(int wpb, const X16Job& a, const X16Job& b, uint32_t blocks, uint32_t blocks_a,
                          uint32_t units, const XGroup* xq, const X16Norm& nrm, const X16Conv& cv,
                          hipStream_t stream) {
    if (xq) {
        if (wpb == 4) {
            HIPLLM_LAUNCH((gemv_x16_pair_kernel<QA, QB, 4, 1>), dim3(blocks), dim3(256), 0, stream, a, b, blocks_a,
                          units, xq, nrm, cv);
        } else {
            HIPLLM_LAUNCH((gemv_x16_pair_kernel<QA, QB, 8, 1>), dim3(blocks), dim3(512), 0, stream, a, b, blocks_a,
                          units, xq, nrm, cv);
        }
        return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
    }
    const size_t lds = static_cast<size_t>(units) * 1024;
    if (wpb == 4) {
        HIPLLM_LAUNCH((gemv_x16_pair_kernel<QA, QB, 4, 3>), dim3(blocks), dim3(256), lds, stream, a, b, blocks_a, units,
                      xq, nrm, cv);
    } else {
        HIPLLM_LAUNCH((gemv_x16_pair_kernel<QA, QB, 8, 3>), dim3(blocks), dim3(512), lds, stream, a, b, blocks_a, units,
                      xq, nrm, cv);
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}
}  // namespace

// Measured shape: one tile per block, 8 waves from 8 units up (one or two
// units per wave), 4 below.
int launch_gemv_x16_pair(uint32_t type_a, const void* packed_a, size_t n_a, float* y_a, uint32_t type_b,
                         const void* packed_b, size_t n_b, float* y_b, size_t k, const float* x, const float* gamma,
                         float eps, const float* conv_w, float* history, size_t ksize, hipStream_t stream,
                         const XGroup* xq, const double* sumsq) {
    if (type_a == kQ8_0) return kInvalidArgument;  // job A: Q4_K or Q6_K
    if ((xq == nullptr) != (sumsq == nullptr)) return kInvalidArgument;
    const XGroup* in = xq ? xq : reinterpret_cast<const XGroup*>(x);  // the input the shared checks see
    int rc = check_x16(type_a, packed_a, in, y_a, n_a, k);
    if (rc == kOk) rc = check_x16(type_b, packed_b, in, y_b, n_b, k);
    if (rc != kOk) return rc;
    if (!xq && (!gamma || reinterpret_cast<uintptr_t>(gamma) % 16 != 0)) return kInvalidArgument;
    if (!(eps > 0.0f) || k > 8192) return kInvalidArgument;
    if (conv_w && (!history || ksize < 2 || ksize > kX16ConvMax)) return kInvalidArgument;
    const uint32_t units = static_cast<uint32_t>(k / 256);
    const uint32_t blocks_a = static_cast<uint32_t>((n_a + 15) / 16), blocks_b = static_cast<uint32_t>((n_b + 15) / 16);
    const X16Job a{static_cast<const uint8_t*>(packed_a), y_a, static_cast<uint32_t>(n_a)};
    const X16Job b{static_cast<const uint8_t*>(packed_b), y_b, static_cast<uint32_t>(n_b)};
    X16Norm nrm{};
    nrm.eps = eps;
    nrm.x_in = x;
    nrm.gamma_in = gamma;
    nrm.sumsq_in = sumsq;
    const X16Conv cv{conv_w, history, static_cast<uint32_t>(n_a), static_cast<uint32_t>(ksize)};
    const int wpb = units >= 8 ? 8 : 4;
    const uint32_t blocks = blocks_a + blocks_b;
    if (type_a == kQ4_K) {
        return type_b == kQ4_K   ? launch_x16_pair_types<kQ4_K, kQ4_K>(wpb, a, b, blocks, blocks_a, units, xq, nrm, cv, stream)
               : type_b == kQ6_K ? launch_x16_pair_types<kQ4_K, kQ6_K>(wpb, a, b, blocks, blocks_a, units, xq, nrm, cv, stream)
                                 : launch_x16_pair_types<kQ4_K, kQ8_0>(wpb, a, b, blocks, blocks_a, units, xq, nrm, cv, stream);
    }
    return type_b == kQ4_K   ? launch_x16_pair_types<kQ6_K, kQ4_K>(wpb, a, b, blocks, blocks_a, units, xq, nrm, cv, stream)
           : type_b == kQ6_K ? launch_x16_pair_types<kQ6_K, kQ6_K>(wpb, a, b, blocks, blocks_a, units, xq, nrm, cv, stream)
                             : launch_x16_pair_types<kQ6_K, kQ8_0>(wpb, a, b, blocks, blocks_a, units, xq, nrm, cv, stream);
}

namespace {
template <uint32_t QT, int MODE, int RTE>
int launch_x16_routed_code(int code, const uint8_t* wp, const uint8_t* wp2, const XGroup* xq, float* y, XGroup* yq,
                           uint32_t nn, uint32_t units, const X16Route& route, hipStream_t stream) {
    const uint32_t tiles = (nn + 15) / 16;
    const X16Norm none{};
    switch (code) {
#define HIPLLM_X16R_CASE(RT, W)                                                                                     \
    case 1000 * RT + 100 + W:                                                                                       \
        HIPLLM_LAUNCH((gemv_x16_kernel<QT, W, RT, MODE, 0, RTE>), dim3((tiles + RT - 1) / RT, route.routes),        \
                      dim3(64 * W), 0, stream, wp, wp2, xq, nullptr, nullptr, y, yq, nn, units, none, route);       \
        break;
        HIPLLM_X16R_CASE(1, 4)
        HIPLLM_X16R_CASE(1, 8)
        HIPLLM_X16R_CASE(2, 4)
        HIPLLM_X16R_CASE(2, 8)
#undef HIPLLM_X16R_CASE
    default:
        return kInvalidArgument;
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

template <uint32_t QT>
int launch_x16_routed_type(int code, const uint8_t* wp, const uint8_t* wp2, const XGroup* xq, float* y, XGroup* yq,
                           uint32_t nn, uint32_t units, const X16Route& route, hipStream_t stream) {
    if (wp2) {
        return route.logits ? launch_x16_routed_code<QT, 1, 2>(code, wp, wp2, xq, y, yq, nn, units, route, stream)
                            : launch_x16_routed_code<QT, 1, 1>(code, wp, wp2, xq, y, yq, nn, units, route, stream);
    }
    return route.logits ? launch_x16_routed_code<QT, 0, 2>(code, wp, wp2, xq, y, yq, nn, units, route, stream)
                        : launch_x16_routed_code<QT, 0, 1>(code, wp, wp2, xq, y, yq, nn, units, route, stream);
}
}  // namespace

// Measured on MI355X (Qwen3.5-35B-A3B expert shapes): 8 waves per block for
// the gate / up pair (512 rows of 2048), two tiles per 4-wave block for the
// down projection (2048 rows of 512: two units per row).
int launch_gemv_x16_routed(uint32_t type, const void* packed, const void* packed2, const XGroup* xq, size_t ldx,
                           int x_routed, float* y, XGroup* yq, size_t ldy, size_t n, size_t k, size_t experts,
                           size_t routes, const int32_t* ids, const float* logits, int32_t* ids_out,
                           float* weights_out, int waves, hipStream_t stream) {
    if (type == kQ8_0) return kInvalidArgument;  // Q4_K / Q6_K expert blocks
    int rc = check_x16(type, packed, xq, y, n, k);
    if (rc == kOk && packed2) rc = check_x16(type, packed2, xq, y, n, k);
    if (rc != kOk) return rc;
    if (n % 16 != 0 || experts == 0 || routes == 0 || routes > 8 || ldx % 16 != 0 || ldx < k || ldy < n) {
        return kInvalidArgument;
    }
    if (yq && (!packed2 || ldy % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0)) return kInvalidArgument;
    if (logits ? (experts > kRouteMaxExperts || !ids_out || !weights_out) : !ids) return kInvalidArgument;
    if (experts > 0xffffffffull || ldx > 0xffffffffull || ldy > 0xffffffffull) return kLengthError;
    const uint32_t units = static_cast<uint32_t>(k / 256), nn = static_cast<uint32_t>(n);
    X16Route route{};
    route.ids = ids;
    route.logits = logits;
    route.ids_out = ids_out;
    route.weights_out = weights_out;
    route.experts = static_cast<uint32_t>(experts);
    route.routes = static_cast<uint32_t>(routes);
    route.expert_bytes = x16_bytes(type, n, k);
    route.x_routed = x_routed ? 1u : 0u;
    route.ldx = static_cast<uint32_t>(ldx);
    route.ldy = static_cast<uint32_t>(ldy);
    const int code = waves ? waves : (units <= 4 ? 2104 : 1108);
    const auto* wp = static_cast<const uint8_t*>(packed);
    const auto* wp2 = static_cast<const uint8_t*>(packed2);
    return type == kQ4_K ? launch_x16_routed_type<kQ4_K>(code, wp, wp2, xq, y, yq, nn, units, route, stream)
                         : launch_x16_routed_type<kQ6_K>(code, wp, wp2, xq, y, yq, nn, units, route, stream);
}

// GEMV over a prepared XGroup input. tiling 0 selects the default.
int launch_gemv_prepped(uint32_t type, const void* w, size_t row_bytes, const float* x, const XGroup* xq,
                        const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                        hipStream_t stream) {
    if (!y) return kInvalidArgument;
    const int rc = check_common(type, w, nullptr, row_bytes, x, xq, n, k);
    if (rc != kOk) return rc;
    const uint32_t units = static_cast<uint32_t>((k + unit_elems(type) - 1) / unit_elems(type));
    const uint32_t nn = static_cast<uint32_t>(n);
    const int code = tiling ? tiling : gemv_pick_shape(type, nn, units, 0);
    if (!valid_tiling(code)) return kInvalidArgument;
    return launch_any<0>(type, code, w, nullptr, row_bytes, x, xq, bias, residual, y, nullptr, nn, units,
                         static_cast<uint32_t>(k / 32), stream);
}

// Fused gate/up GEMV + SwiGLU: y = silu(Wg x) * (Wu x); yq (optional,
// n % 16 == 0) receives the XGroup form of y for the down projection.
int launch_gemv_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                       const XGroup* xq, float* y, XGroup* yq, size_t n, size_t k, int tiling, hipStream_t stream) {
    if (!wu || !y) return kInvalidArgument;
    const int rc = check_common(type, wg, wu, row_bytes, x, xq, n, k);
    if (rc != kOk) return rc;
    if (yq && (n % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0)) return kInvalidArgument;
    const uint32_t units = static_cast<uint32_t>((k + unit_elems(type) - 1) / unit_elems(type));
    const uint32_t nn = static_cast<uint32_t>(n);
    const int code = tiling ? tiling : gemv_pick_shape(type, nn, units, 1);
    if (!valid_tiling(code) || (yq && !writes_whole_groups(code))) return kInvalidArgument;
    return launch_any<1>(type, code, wg, wu, row_bytes, x, xq, nullptr, nullptr, y, yq, nn, units,
                         static_cast<uint32_t>(k / 32), stream);
}

// The NORM tiling nearest a plain pick: 2 or 4 rows per octet, 8 or 16
// octets per row group (204 / 408 for a SwiGLU with XGroup output).
static int norm_tiling(int t, int mode, bool whole_groups) {
    if (mode == 1 && whole_groups) return t == 408 ? 408 : 204;
    const int R = t / 100 >= 4 ? 4 : 2;
    const int OPR = t % 100 >= 16 ? 16 : 8;
    return 100 * R + OPR;
}

// gamma nullptr: no norm, the prologue only encodes x (eps unused).
static bool norm_ok(uint32_t type, const float* x, const float* gamma, size_t k, float eps) {
    return (type == kQ4_K || type == kQ6_K || type == kQ8_0 || type == kQ5_0) && x && k % 16 == 0 &&
           k / 16 <= kNormMaxGroups && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(gamma) % 16 == 0 && (!gamma || eps > 0.0f);
}

// y = W rmsnorm(x) (+ bias) (+ residual) with the norm in the GEMV's
// prologue (quantized weights; k <= 8192); without gamma, y = W x with x's
// XGroup form made in the prologue.
int launch_gemv_norm(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* gamma, float eps,
                     const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                     hipStream_t stream) {
    if (!y) return kInvalidArgument;
    if (!norm_ok(type, x, gamma, k, eps)) return kInvalidArgument;
    const int rc = check_common(type, w, nullptr, row_bytes, x, nullptr, n, k);
    if (rc != kOk && rc != kInvalidArgument) return rc;
    if (!w || row_bytes < k / block_elems(type) * block_bytes(type)) return kInvalidArgument;
    const uint32_t units = static_cast<uint32_t>((k + unit_elems(type) - 1) / unit_elems(type));
    const uint32_t nn = static_cast<uint32_t>(n);
    const int code = tiling ? tiling : norm_tiling(gemv_pick_shape(type, nn, units, 0), 0, false);
    return launch_any_norm<0>(type, code, w, nullptr, row_bytes, x, gamma, eps, bias, residual, y, nullptr, nn, units,
                              static_cast<uint32_t>(k / 32), stream);
}

// y = silu(Wg rmsnorm(x)) * (Wu rmsnorm(x)), yq (optional) its XGroup form,
// with the norm in the prologue.
int launch_gemv_swiglu_norm(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                            const float* gamma, float eps, float* y, XGroup* yq, size_t n, size_t k, int tiling,
                            hipStream_t stream) {
    if (!wg || !wu || !y) return kInvalidArgument;
    if (!norm_ok(type, x, gamma, k, eps)) return kInvalidArgument;
    if (row_bytes < k / block_elems(type) * block_bytes(type)) return kInvalidArgument;
    if (n == 0 || n > 0x7fffffffull || k == 0 || k % block_elems(type) != 0) return kInvalidArgument;
    if (yq && (n % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0)) return kInvalidArgument;
    const uint32_t units = static_cast<uint32_t>((k + unit_elems(type) - 1) / unit_elems(type));
    const uint32_t nn = static_cast<uint32_t>(n);
    const int code = tiling ? tiling : norm_tiling(gemv_default_tiling(nn, units, 1, 1, yq != nullptr), 1, yq != nullptr);
    return launch_any_norm<1>(type, code, wg, wu, row_bytes, x, gamma, eps, nullptr, nullptr, y, yq, nn, units,
                              static_cast<uint32_t>(k / 32), stream);
}

// y = residual + (sum_q weights[q] down[q] + sigmoid(sgate[0]) W x) for one
// token, x raw FP32 (its XGroup form made in the prologue).
int launch_gemv_moe_combine(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* residual,
                            const float* down, const float* weights, const float* sgate, size_t routes, float* y,
                            size_t n, size_t k, hipStream_t stream) {
    if (!y || !residual || !down || !weights || !sgate || routes == 0 || routes > kCombineRoutes) {
        return kInvalidArgument;
    }
    if (!norm_ok(type, x, nullptr, k, 0.0f)) return kInvalidArgument;
    if (!w || row_bytes < k / block_elems(type) * block_bytes(type) || k % block_elems(type) != 0) {
        return kInvalidArgument;
    }
    if ((type == kQ4_K && (row_bytes % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 16 != 0)) ||
        row_bytes % 2 != 0 || reinterpret_cast<uintptr_t>(w) % 2 != 0) {
        return kInvalidArgument;
    }
    if (n == 0 || n > 0x7fffffffull) return n == 0 ? kInvalidArgument : kLengthError;
    const uint32_t units = static_cast<uint32_t>((k + unit_elems(type) - 1) / unit_elems(type));
    const uint32_t nn = static_cast<uint32_t>(n);
    const int code = norm_tiling(gemv_pick_shape(type, nn, units, 0), 0, false);
    MoeCombine c;
    c.down = down;
    c.weights = weights;
    c.sgate = sgate;
    c.routes = static_cast<uint32_t>(routes);
    return launch_any_norm<2>(type, code, w, nullptr, row_bytes, x, nullptr, 0.0f, nullptr, residual, y, nullptr, nn,
                              units, static_cast<uint32_t>(k / 32), stream, c);
}

// One wave's products of a 16-row x16 tile (units tile-units from wt) with
// an XGroup input row whose unit u is the 1 KiB at xg + 1024 u (global, or
// LDS when x_lds): two units in flight, each unit's groups stored to the
// wave's 1 KiB of LDS (global input) and read as the MFMA A slices; lanes r,
// r + 16, r + 32, r + 48 then hold row r's four partial sums, returned
// summed in lanes r < 16. lds: the wave's 2 KiB (input slot, zero region).
// pro() runs once the first two units' loads are issued.
template <uint32_t QT, typename Pro>
__device__ __forceinline__ float x16_wave_tile(const uint8_t* __restrict__ wt, const uint8_t* xg, bool x_lds,
                                               uint32_t units, uint8_t* lds, uint32_t lane, Pro pro) {
    using F = X16<QT>;
    constexpr uint32_t kTileUnit = 16 * F::kBlock;
    const uint32_t r = lane & 15, s = lane >> 4;
    if (lane < kMfmaZeroBytes / 16) *reinterpret_cast<uint4*>(lds + 1024 + 16 * lane) = make_uint4(0, 0, 0, 0);
    const bool a_lane = (r >> 2) == s && (r & 3) < 3;
    const uint32_t slot = F::group_base(s);
    struct Slot {
        uint4 x;
        typename F::Unit w;
    };
    auto fill = [&](Slot& d, uint32_t u) {
        if (!x_lds) d.x = reinterpret_cast<const uint4*>(xg + 1024 * u)[lane];
        d.w = F::load(wt + static_cast<size_t>(u) * kTileUnit, r, s, lane);
    };
    auto consume = [&](const Slot& d, uint32_t u, float acc) {
        const uint8_t* base = lds;
        if (x_lds) {
            base = xg + 1024 * u;
        } else {
            *reinterpret_cast<uint4*>(lds + 16 * lane) = d.x;
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
        const uint8_t* a_src = a_lane ? base + slot + 16 * (r & 3) : lds + 1024;
        acc = F::unit(d.w, a_src, base + slot + 48, r, s, acc);
        if (!x_lds) {
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
        return acc;
    };
    Slot s0, s1;
    if (units > 0) fill(s0, 0);
    if (units > 1) fill(s1, 1);
    pro();
    float acc = 0.0f;
    for (uint32_t u = 0; u < units; u += 2) {
        acc = consume(s0, u, acc);
        if (u + 2 < units) fill(s0, u + 2);
        if (u + 1 < units) {
            acc = consume(s1, u + 1, acc);
            if (u + 3 < units) fill(s1, u + 3);
        }
    }
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    return acc;
}

// The routed expert down projections of one token, the shared expert's down
// projection and the MoE combine in one launch. Block = 16-row tile of the
// output; wave j < routes multiplies the tile of expert ids[j] (clamped to
// experts - 1) in the x16 copy of the whole down block by route j's SwiGLU
// output (XGroup row j, ldx values apart), wave `routes` the shared expert's
// tile by its SwiGLU output, which arrives as FP32 (sx, k_s values) and is
// encoded into LDS by that wave. Epilogue (thread r < 16), the expression of
// the vector combine: y = residual + (sum_j weights[j] down_j (route order)
// + shared * sigmoid(sgate[0])).
constexpr uint32_t kMoeDownMaxShared = 2048;  // shared-expert inner size held in LDS

// nrm.gamma_out (nullable): each tile also writes the next RMSNorm's data as
// an x16 NORM 2 launch does (the XGroup form of y * gamma_out into
// nrm.yq_out, the double sum of squares of its 16 values in row order into
// nrm.sumsq_out).
template <uint32_t QR, uint32_t QS>
__global__ __launch_bounds__(64 * (kCombineRoutes + 1)) void x16_moe_down_kernel(
    const uint8_t* __restrict__ down_x16, size_t expert_bytes, const int32_t* __restrict__ ids, uint32_t experts,
    const XGroup* __restrict__ xq, uint32_t ldx, uint32_t units_r, const uint8_t* __restrict__ shared_x16,
    const float* __restrict__ sx, uint32_t units_s, const float* __restrict__ weights,
    const float* __restrict__ sgate, const float* __restrict__ residual, float* __restrict__ y, uint32_t n,
    uint32_t routes, const X16Norm nrm) {
    __shared__ __align__(16) uint8_t xs[kCombineRoutes + 1][2048];
    __shared__ __align__(16) XGroup sxg[kMoeDownMaxShared / 16];
    __shared__ float vals[kCombineRoutes + 1][16];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t tile = blockIdx.x, row = tile * 16 + threadIdx.x;
    // Epilogue operands, loaded now.
    float res = 0.0f, sg = 0.0f, gam = 0.0f, wts[kCombineRoutes];
    if (threadIdx.x < 16) {
        if (row < n) res = residual[row];
        if (nrm.gamma_out && row < n) gam = nrm.gamma_out[row];
        sg = sgate[0];
#pragma unroll
        for (uint32_t q = 0; q < kCombineRoutes; ++q) wts[q] = q < routes ? weights[q] : 0.0f;
    }
    float v = 0.0f;
    if (wave < routes) {
        const uint32_t e = min(static_cast<uint32_t>(ids[wave]), experts - 1);
        const uint8_t* wt = down_x16 + static_cast<size_t>(e) * expert_bytes +
                            static_cast<size_t>(tile) * units_r * (16 * X16<QR>::kBlock);
        v = x16_wave_tile<QR>(wt, reinterpret_cast<const uint8_t*>(xq + static_cast<size_t>(wave) * (ldx / 16)),
                              false, units_r, xs[wave], lane, [] {});
    } else if (wave == routes) {
        const uint8_t* wt = shared_x16 + static_cast<size_t>(tile) * units_s * (16 * X16<QS>::kBlock);
        // The input's XGroup form is made while the first weight loads fly.
        v = x16_wave_tile<QS>(wt, reinterpret_cast<const uint8_t*>(sxg), true, units_s, xs[wave], lane, [&] {
            for (uint32_t g = lane; g < 16 * units_s; g += 64) xgroup_encode_from(sx + 16 * g, sxg + g);
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        });
    }
    if (wave <= routes && lane < 16) vals[wave][lane] = v;
    __syncthreads();
    if (threadIdx.x < 16 && row < n) {
        float acc = 0.0f;
#pragma unroll
        for (uint32_t q = 0; q < kCombineRoutes; ++q) {
            if (q < routes) acc += wts[q] * vals[q][threadIdx.x];
        }
        float moe = acc;
        moe += vals[routes][threadIdx.x] * sigmoid_ref(sg);
        const float out = res + moe;
        y[row] = out;
        vals[0][threadIdx.x] = out * gam;  // each thread rewrites its own slots after reading them
        vals[1][threadIdx.x] = out;
    }
    if (nrm.gamma_out) {
        __syncthreads();
        if (threadIdx.x == 0) {
            xgroup_encode_from(vals[0], nrm.yq_out + tile);
            double ss = 0.0;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const double t = vals[1][i];
                ss += t * t;
            }
            nrm.sumsq_out[tile] = ss;
        }
    }
}

int launch_x16_moe_down(uint32_t type_r, const void* down_x16, const int32_t* ids, size_t experts, const XGroup* xq,
                        size_t ldx, size_t k_r, uint32_t type_s, const void* shared_x16, const float* sx, size_t k_s,
                        const float* weights, const float* sgate, const float* residual, float* y, size_t n,
                        size_t routes, hipStream_t stream, const X16Norm* norm_out) {
    if (!down_x16 || !ids || !xq || !shared_x16 || !sx || !weights || !sgate || !residual || !y || experts == 0 ||
        routes == 0 || routes > kCombineRoutes || n == 0 || n % 16 != 0) {
        return kInvalidArgument;
    }
    if ((type_r != kQ4_K && type_r != kQ6_K) || !x16_type(type_s)) return kInvalidArgument;
    if (k_r == 0 || k_r % 256 != 0 || k_s == 0 || k_s % 256 != 0 || k_s > kMoeDownMaxShared || ldx < k_r ||
        ldx % 16 != 0) {
        return kInvalidArgument;
    }
    for (const void* p : {static_cast<const void*>(down_x16), static_cast<const void*>(xq), shared_x16,
                          static_cast<const void*>(sx)}) {
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return kInvalidArgument;
    }
    X16Norm nrm{};
    if (norm_out && norm_out->gamma_out) {
        if (!norm_out->yq_out || !norm_out->sumsq_out || reinterpret_cast<uintptr_t>(norm_out->yq_out) % 16 != 0) {
            return kInvalidArgument;
        }
        nrm.gamma_out = norm_out->gamma_out;
        nrm.yq_out = norm_out->yq_out;
        nrm.sumsq_out = norm_out->sumsq_out;
    }
    if (n > 0x7fffffffull || experts > 0xffffffffull || ldx > 0xffffffffull) return kLengthError;
    const size_t expert_bytes = x16_bytes(type_r, n, k_r);
    const uint32_t ur = static_cast<uint32_t>(k_r / 256), us = static_cast<uint32_t>(k_s / 256);
    const dim3 grid(static_cast<uint32_t>(n / 16)), block(static_cast<uint32_t>(64 * (routes + 1)));
    const auto* dw = static_cast<const uint8_t*>(down_x16);
    const auto* sw = static_cast<const uint8_t*>(shared_x16);
    const uint32_t E = static_cast<uint32_t>(experts), nn = static_cast<uint32_t>(n), R = static_cast<uint32_t>(routes),
                   lx = static_cast<uint32_t>(ldx);
#define HIPLLM_MOE_DOWN(QR, QS)                                                                                    \
    HIPLLM_LAUNCH((x16_moe_down_kernel<QR, QS>), grid, block, 0, stream, dw, expert_bytes, ids, E, xq, lx, ur, sw, sx, \
                  us, weights, sgate, residual, y, nn, R, nrm)
    if (type_r == kQ4_K) {
        if (type_s == kQ4_K) {
            HIPLLM_MOE_DOWN(kQ4_K, kQ4_K);
        } else if (type_s == kQ6_K) {
            HIPLLM_MOE_DOWN(kQ4_K, kQ6_K);
        } else {
            HIPLLM_MOE_DOWN(kQ4_K, kQ8_0);
        }
    } else {
        if (type_s == kQ4_K) {
            HIPLLM_MOE_DOWN(kQ6_K, kQ4_K);
        } else if (type_s == kQ6_K) {
            HIPLLM_MOE_DOWN(kQ6_K, kQ6_K);
        } else {
            HIPLLM_MOE_DOWN(kQ6_K, kQ8_0);
        }
    }
#undef HIPLLM_MOE_DOWN
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

// Routed expert vectors of a short prompt grouped by expert (route groups of
// at most kX16GroupRows vectors, launch_route_groups): block (tile, group)
// reads its expert's 16-row tile of the x16 copy of the whole expert block
// once and multiplies it by every vector of the group. Vector j of the group
// is routed vector order[first + j] (its input row: that index when
// x_routed, else the index / routes; its output row: that index). WPB waves
// (4, or 2 for rows of at most two units) split the units; per unit a wave
// loads the weights (both matrices for the
// SwiGLU pair) and each vector's 1 KiB of input groups, then runs the
// unit's MFMAs for each vector from its own LDS slot. MODE 0: y = W x;
// MODE 1: y = silu(Wg x) * (Wu x) and yq its XGroup form (one group per
// tile). Groups past *ngroups exit at once.
template <uint32_t QT, int MODE, int WPB>
__global__ __launch_bounds__(64 * WPB) void x16_grouped_kernel(
    const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, size_t expert_bytes, uint32_t experts,
    const XGroup* __restrict__ xq, uint32_t ldx, uint32_t x_routed, uint32_t routes, float* __restrict__ y,
    XGroup* __restrict__ yq, uint32_t ldy, uint32_t n, uint32_t units, const int32_t* __restrict__ order,
    const int32_t* __restrict__ groups, const uint32_t* __restrict__ ngroups) {
    constexpr int VB = kX16GroupRows, NM = MODE == 1 ? 2 : 1;
    using F = X16<QT>;
    constexpr uint32_t kTileUnit = 16 * F::kBlock;
    if (blockIdx.y >= *ngroups) return;
    const uint32_t first = static_cast<uint32_t>(groups[2 * blockIdx.y]);
    const uint32_t packed = static_cast<uint32_t>(groups[2 * blockIdx.y + 1]);
    const uint32_t e = min(packed & 0xffffu, experts - 1);
    const uint32_t cnt = min(packed >> 16, static_cast<uint32_t>(VB));  // launch_route_groups with vmax <= VB
    const uint32_t tile = blockIdx.x;
    __shared__ __align__(16) uint8_t xs[WPB][VB + 1][1024];  // per wave: one slot per vector, then zeros
    __shared__ float part[WPB][VB][NM][16];
    __shared__ __align__(16) float outs[VB][16];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t r = lane & 15, s = lane >> 4;
    const uint8_t* wt[NM];
    wt[0] = w + static_cast<size_t>(e) * expert_bytes + static_cast<size_t>(tile) * units * kTileUnit;
    if (MODE == 1) wt[NM - 1] = w2 + static_cast<size_t>(e) * expert_bytes + static_cast<size_t>(tile) * units * kTileUnit;
    uint32_t vec[VB];
    const uint4* xrow[VB];
#pragma unroll
    for (int j = 0; j < VB; ++j) {
        vec[j] = j < static_cast<int>(cnt) ? static_cast<uint32_t>(order[first + j]) : 0u;
        const uint32_t src = x_routed ? vec[j] : vec[j] / routes;
        xrow[j] = reinterpret_cast<const uint4*>(xq + static_cast<size_t>(src) * (ldx / 16));
    }
    uint8_t* zero = xs[wave][VB];
    for (uint32_t i = lane; i < kMfmaZeroBytes / 16; i += 64) reinterpret_cast<uint4*>(zero)[i] = make_uint4(0, 0, 0, 0);
    const bool a_lane = (r >> 2) == s && (r & 3) < 3;
    const uint32_t slot = F::group_base(s);
    float acc[VB][NM];
#pragma unroll
    for (int j = 0; j < VB; ++j)
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[j][m] = 0.0f;
    for (uint32_t u = wave; u < units; u += WPB) {
        typename F::Unit wu[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) wu[m] = F::load(wt[m] + static_cast<size_t>(u) * kTileUnit, r, s, lane);
        uint4 xv[VB];
#pragma unroll
        for (int j = 0; j < VB; ++j) xv[j] = j < static_cast<int>(cnt) ? xrow[j][64 * u + lane] : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < VB; ++j) *reinterpret_cast<uint4*>(xs[wave][j] + 16 * lane) = xv[j];
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int j = 0; j < VB; ++j) {
            if (j < static_cast<int>(cnt)) {
                const uint8_t* a_src = a_lane ? xs[wave][j] + slot + 16 * (r & 3) : zero;
#pragma unroll
                for (int m = 0; m < NM; ++m) acc[j][m] = F::unit(wu[m], a_src, xs[wave][j] + slot + 48, r, s, acc[j][m]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int j = 0; j < VB; ++j) {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            float v = acc[j][m];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            if (lane < 16) part[wave][j][m][lane] = v;
        }
    }
    __syncthreads();
    if (tid < 16 * cnt) {
        const uint32_t j = tid / 16, rr = tid % 16, row = tile * 16 + rr;
        float v = part[0][j][0][rr];
#pragma unroll
        for (int i = 1; i < WPB; ++i) v += part[i][j][0][rr];
        if (MODE == 1) {
            float g2 = part[0][j][NM - 1][rr];
#pragma unroll
            for (int i = 1; i < WPB; ++i) g2 += part[i][j][NM - 1][rr];
            v = row < n ? silu_mul(v, g2) : 0.0f;
            outs[j][rr] = v;
        }
        if (row < n) y[static_cast<size_t>(order[first + j]) * ldy + row] = v;
    }
    if (MODE == 1 && yq) {
        __syncthreads();
        if (tid < cnt && tile * 16 < n) {
            xgroup_encode_from(outs[tid], yq + static_cast<size_t>(order[first + tid]) * (ldy / 16) + tile);
        }
    }
}

int launch_x16_grouped(uint32_t type, const void* packed, const void* packed2, const XGroup* xq, size_t ldx,
                       int x_routed, size_t routes, float* y, XGroup* yq, size_t ldy, size_t n, size_t k,
                       size_t experts, const int32_t* order, const int32_t* groups, const uint32_t* ngroups,
                       size_t max_groups, hipStream_t stream) {
    if (type != kQ4_K && type != kQ6_K) return kInvalidArgument;
    int rc = check_x16(type, packed, xq, y, n, k);
    if (rc == kOk && packed2) rc = check_x16(type, packed2, xq, y, n, k);
    if (rc != kOk) return rc;
    if (n % 16 != 0 || experts == 0 || routes == 0 || !order || !groups || !ngroups || max_groups == 0 ||
        ldx % 16 != 0 || ldx < k || ldy < n) {
        return kInvalidArgument;
    }
    if (yq && (!packed2 || ldy % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0)) return kInvalidArgument;
    if (max_groups > 65535 || experts > 0xffffffffull || ldx > 0xffffffffull || ldy > 0xffffffffull) {
        return kLengthError;
    }
    const size_t expert_bytes = x16_bytes(type, n, k);
    const dim3 grid(static_cast<uint32_t>(n / 16), static_cast<uint32_t>(max_groups));
    const auto* wp = static_cast<const uint8_t*>(packed);
    const auto* wp2 = static_cast<const uint8_t*>(packed2);
    const uint32_t E = static_cast<uint32_t>(experts), lx = static_cast<uint32_t>(ldx), xr = x_routed ? 1u : 0u,
                   R = static_cast<uint32_t>(routes), ly = static_cast<uint32_t>(ldy), nn = static_cast<uint32_t>(n),
                   units = static_cast<uint32_t>(k / 256);
#define HIPLLM_X16G(QT, M)                                                                                          \
    if (units <= 2) {                                                                                               \
        HIPLLM_LAUNCH((x16_grouped_kernel<QT, M, 2>), grid, dim3(128), 0, stream, wp, wp2, expert_bytes, E, xq, lx, xr, \
                      R, y, yq, ly, nn, units, order, groups, ngroups);                                              \
    } else {                                                                                                        \
        HIPLLM_LAUNCH((x16_grouped_kernel<QT, M, 4>), grid, dim3(256), 0, stream, wp, wp2, expert_bytes, E, xq, lx, xr, \
                      R, y, yq, ly, nn, units, order, groups, ngroups);                                              \
    }
    if (type == kQ4_K) {
        if (packed2) {
            HIPLLM_X16G(kQ4_K, 1);
        } else {
            HIPLLM_X16G(kQ4_K, 0);
        }
    } else {
        if (packed2) {
            HIPLLM_X16G(kQ6_K, 1);
        } else {
            HIPLLM_X16G(kQ6_K, 0);
        }
    }
#undef HIPLLM_X16G
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

// Routed expert gate/up + SwiGLU with the routes chosen in every block's
// prologue (Batch, ROUTE): 16-row blocks, 2 rows x 4 octets, or 4 x 8 from
// 8192 rows on.
template <uint32_t T>
int launch_routed(const void* wg, const void* wu, size_t row_bytes, const float* x, const XGroup* xq, float* y,
                  XGroup* yq, uint32_t n, uint32_t units, uint32_t kblocks, const Batch& b, uint32_t vectors,
                  hipStream_t stream) {
    const auto* wp = static_cast<const uint8_t*>(wg);
    const auto* up = static_cast<const uint8_t*>(wu);
    if (n >= 8192) {
        HIPLLM_LAUNCH((gemv_kernel<T, 4, 8, 1, false, true>), dim3((n + 15) / 16, vectors), dim3(256), 0, stream,
                           wp, up, row_bytes, x, xq, nullptr, nullptr, y, yq, n, units, kblocks, b);
    } else {
        HIPLLM_LAUNCH((gemv_kernel<T, 2, 4, 1, false, true>), dim3((n + 15) / 16, vectors), dim3(256), 0, stream,
                           wp, up, row_bytes, x, xq, nullptr, nullptr, y, yq, n, units, kblocks, b);
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

int launch_gemv_routed_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                              const XGroup* xq, size_t ldx, float* y, XGroup* yq, size_t n, size_t k, size_t tokens,
                              const float* logits, size_t ld_logits, size_t experts, size_t routes,
                              size_t expert_stride, int32_t* ids_out, float* weights_out, hipStream_t stream) {
    if (!y || !wu || !logits || !ids_out || !weights_out || tokens == 0) return kInvalidArgument;
    if (!(type == kQ4_K || type == kQ6_K || type == kQ8_0 || type == kQ5_0)) return kInvalidArgument;
    const int rc = check_common(type, wg, wu, row_bytes, x, xq, n, k, expert_stride);
    if (rc != kOk) return rc;
    if (experts == 0 || routes == 0 || routes > 8 || routes > experts || ld_logits < experts ||
        expert_stride < n * row_bytes || ldx < k || ldx % 16 != 0) {
        return kInvalidArgument;
    }
    if (yq && (n % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0)) return kInvalidArgument;
    if (experts > kRouteMaxExperts) return kLengthError;
    if (tokens * routes > 65535 || ldx > 0xffffffffu || ld_logits > 0xffffffffu) return kLengthError;
    Batch b;
    b.experts = static_cast<uint32_t>(experts);
    b.routes = static_cast<uint32_t>(routes);
    b.expert_stride = expert_stride;
    b.ldx = static_cast<uint32_t>(ldx);
    b.ldy = static_cast<uint32_t>(n);
    b.logits = logits;
    b.ld_logits = static_cast<uint32_t>(ld_logits);
    b.ids_out = ids_out;
    b.weights_out = weights_out;
    const uint32_t units = static_cast<uint32_t>((k + unit_elems(type) - 1) / unit_elems(type));
    const uint32_t nn = static_cast<uint32_t>(n), kb = static_cast<uint32_t>(k / 32);
    const uint32_t nv = static_cast<uint32_t>(tokens * routes);
    switch (type) {
    case kQ4_K: return launch_routed<kQ4_K>(wg, wu, row_bytes, x, xq, y, yq, nn, units, kb, b, nv, stream);
    case kQ6_K: return launch_routed<kQ6_K>(wg, wu, row_bytes, x, xq, y, yq, nn, units, kb, b, nv, stream);
    case kQ8_0: return launch_routed<kQ8_0>(wg, wu, row_bytes, x, xq, y, yq, nn, units, kb, b, nv, stream);
    default: return launch_routed<kQ5_0>(wg, wu, row_bytes, x, xq, y, yq, nn, units, kb, b, nv, stream);
    }
}

int launch_gemv_multi_norm(const GemvJob* jobs, size_t count, const float* x, const float* gamma, float eps, size_t k,
                           float* norm, XGroup* normq, hipStream_t stream) {
    if (!jobs || count == 0 || count > kMultiJobs) return kInvalidArgument;
    if (!x || !gamma || !(eps > 0.0f) || k == 0 || k % 32 != 0 || k / 16 > kNormMaxGroups) return kInvalidArgument;
    for (const void* p : {static_cast<const void*>(x), static_cast<const void*>(gamma), static_cast<const void*>(norm),
                          static_cast<const void*>(normq)}) {
        if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return kInvalidArgument;  // nullptr passes
    }
    if (normq && !norm) return kInvalidArgument;
    GemvMulti m{};
    uint64_t total = 0;
    uint32_t heavy = 0;
    for (size_t i = 0; i < count; ++i) {
        GemvJob j = jobs[i];
        const bool quant = j.type == kQ4_K || j.type == kQ6_K || j.type == kQ8_0 || j.type == kQ5_0;
        if (!j.y || (j.mode != 0 && j.mode != 1) || !(quant || (j.type == kF32 && j.mode == 0))) {
            return kInvalidArgument;
        }
        // The input comes from the prologue: x stands in for the XGroup pointer in the shared checks.
        const int rc = check_common(j.type, j.w, j.mode ? j.w2 : nullptr, j.row_bytes, x,
                                    reinterpret_cast<const XGroup*>(x), j.n, k);
        if (rc != kOk) return rc;
        if (j.mode == 1 && (!j.w2 || j.bias || j.residual)) return kInvalidArgument;
        if (j.yq && (j.mode != 1 || j.n % 16 != 0 || reinterpret_cast<uintptr_t>(j.yq) % 16 != 0)) {
            return kInvalidArgument;
        }
        if (j.type == kQ6_K) heavy |= j.mode ? kMultiQ6KSwiGLU : kMultiQ6K;
        const int t = multi_tiling(j.type, j.mode == 0 ? 0 : (j.yq ? 1 : 2));
        const uint32_t rpb = 32u / (t % 100) * (t / 100);
        j.blocks = (j.n + rpb - 1) / rpb;
        total += j.blocks;
        m.job[i] = j;
    }
    if (total > 0x7fffffffull) return kLengthError;
    m.jobs = static_cast<uint32_t>(count);
    m.kblocks = static_cast<uint32_t>(k / 32);
    m.x = x;
    m.gamma = gamma;
    m.eps = eps;
    m.norm = norm;
    m.normq = normq;
    auto kernel = heavy == 0 ? gemv_multi_kernel<0>
                  : heavy == kMultiQ6K ? gemv_multi_kernel<kMultiQ6K> : gemv_multi_kernel<kMultiQ6K | kMultiQ6KSwiGLU>;
    HIPLLM_LAUNCH(kernel, dim3(static_cast<uint32_t>(total)), dim3(256), k * 4, stream, m);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

// A batch of GEMVs through one matrix or through routed experts (see Batch):
// vector j computes y[j, :n] = W_j x_j (+ bias) (+ residual[j]) or, with
// wu != nullptr, y[j] = silu(Wg_j x_j) * (Wu_j x_j) with optional yq[j].
int launch_gemv_batched(uint32_t type, const void* w, const void* wu, size_t row_bytes, const float* x,
                        const XGroup* xq, const float* bias, const float* residual, float* y, XGroup* yq, size_t n,
                        size_t k, size_t vectors, const int32_t* ids, size_t experts, size_t routes,
                        size_t expert_stride, int x_routed, size_t ldx, size_t ldy, hipStream_t stream) {
    if (!y || vectors == 0) return kInvalidArgument;
    const int rc = check_common(type, w, wu, row_bytes, x, xq, n, k, ids ? expert_stride : 0);
    if (rc != kOk) return rc;
    if (ldx < k || ldx % 16 != 0 || ldy < n) return kInvalidArgument;
    if (ids && (experts == 0 || routes == 0 || expert_stride < n * row_bytes)) return kInvalidArgument;
    if (!ids && routes == 0) return kInvalidArgument;
    if (yq && (!wu || n % 16 != 0 || ldy % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0)) {
        return kInvalidArgument;
    }
    if (wu && (bias || residual)) return kInvalidArgument;
    if (vectors > 65535 || ldx > 0xffffffffu || ldy > 0xffffffffu || experts > 0xffffffffu ||
        routes > 0xffffffffu) {
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
    const uint32_t units = static_cast<uint32_t>((k + unit_elems(type) - 1) / unit_elems(type));
    const uint32_t nn = static_cast<uint32_t>(n);
    const uint32_t nv = static_cast<uint32_t>(vectors);
    const uint32_t kb = static_cast<uint32_t>(k / 32);
    if (!wu) {
        const int t = gemv_default_tiling(nn, units, 0, nv);
        return launch_any<0>(type, t, w, nullptr, row_bytes, x, xq, bias, residual, y, nullptr, nn, units, kb, stream,
                             b, nv);
    }
    const int t = gemv_default_tiling(nn, units, 1, nv, yq != nullptr);
    return launch_any<1>(type, t, w, wu, row_bytes, x, xq, nullptr, nullptr, y, yq, nn, units, kb, stream, b, nv);
}

}  // namespace hipllm
