// Router pieces shared by the router kernel and the expert GEMV that routes
// in its prologue: the reference's sign-branched sigmoid and the per-token
// softmax / top-k / renormalisation by one wave.
//
// Reference semantics: softmax metal_llm.metal:826-890, top-k insertion
// 1424-1459 (strict '>': lower expert id wins ties), renorm 1461-1474,
// sigmoid 1186-1197.
#pragma once

#include "common.h"

namespace hipllm {

// Sign-branched sigmoid of the reference (metal_llm.metal:1186-1197).
__device__ __forceinline__ float sigmoid_ref(float v) {
    return v >= 0.0f ? 1.0f / (1.0f + expf(-v)) : expf(v) / (1.0f + expf(v));
}

// One 64-lane wave per token, expert e held by lane e % 64 in register e / 64
// (PL registers per lane, PL = 4 covers 256 experts): softmax with wave
// reductions, then k rounds of a wave-wide maximum over 64-bit keys
// (probability bits + 1 in the high word, the complemented expert id in the
// low word, 0 for removed, NaN or absent experts), so one unsigned compare
// orders by probability and, on equal probabilities, keeps the lower id.
// Taking maxima in descending order with lower-id tie-breaks selects exactly
// what the reference's insertion scan with a strict '>' keeps, in the same
// rank order. The winner's register is cleared in its lane; no LDS, no
// barriers, DPP and v_readlane only.
constexpr uint32_t kMaxExperts = 1024;

__device__ __forceinline__ uint64_t wave_max_key(uint64_t key) {
    auto step = [&](uint64_t other) { key = other > key ? other : key; };
    auto mov = [](uint64_t v, auto ctrl) {
        constexpr int c = decltype(ctrl)::value;
        return static_cast<uint64_t>(dpp_u32<c>(static_cast<uint32_t>(v))) |
               (static_cast<uint64_t>(dpp_u32<c>(static_cast<uint32_t>(v >> 32))) << 32);
    };
    step(mov(key, std::integral_constant<int, kDppQuadXor1>{}));
    step(mov(key, std::integral_constant<int, kDppQuadXor2>{}));
    step(mov(key, std::integral_constant<int, kDppHalfMirror>{}));
    step(mov(key, std::integral_constant<int, kDppMirror>{}));
    auto at = [&](int lane) {
        return static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), lane))) |
               (static_cast<uint64_t>(static_cast<uint32_t>(
                    __builtin_amdgcn_readlane(static_cast<int>(key >> 32), lane))) << 32);
    };
    const uint64_t a = at(0), b = at(16), c = at(32), d = at(48);
    const uint64_t ab = a > b ? a : b, cd = c > d ? c : d;
    return ab > cd ? ab : cd;
}

// Softmax, top-k and renormalisation of one token's logits by one wave
// (lane = the lane in that wave); writes k ids and weights.
template <uint32_t PL>
__device__ __forceinline__ void topk_row(const float* row, uint32_t experts, uint32_t k, int32_t* __restrict__ ids,
                                         float* __restrict__ weights, uint32_t lane) {
    float p[PL];
    float m = -INFINITY;
#pragma unroll
    for (uint32_t r = 0; r < PL; ++r) {
        const uint32_t e = lane + 64 * r;
        p[r] = e < experts ? row[e] : -INFINITY;
        m = fmaxf(m, p[r]);
    }
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (uint32_t r = 0; r < PL; ++r) {
        p[r] = p[r] == -INFINITY ? 0.0f : expf(p[r] - m);
        s += lane + 64 * r < experts ? p[r] : 0.0f;
    }
    s = wave_sum(s);
    uint32_t key_hi[PL];  // probability bits + 1; 0 = not selectable
#pragma unroll
    for (uint32_t r = 0; r < PL; ++r) {
        // Probabilities are >= +0, so their bit patterns order like the values.
        const float v = s > 0.0f ? p[r] / s : 0.0f;
        key_hi[r] = (lane + 64 * r < experts && v == v) ? __float_as_uint(v) + 1u : 0u;
    }
    float my_v = 0.0f;  // lane r keeps the weight of rank r
    uint32_t my_i = 0;
    for (uint32_t rank = 0; rank < k; ++rank) {
        uint32_t bh = 0, bi = 0xffffffffu;
#pragma unroll
        for (uint32_t r = 0; r < PL; ++r) {
            if (key_hi[r] > bh) {  // ids increase with r, so '>' keeps the lower id on ties
                bh = key_hi[r];
                bi = lane + 64 * r;
            }
        }
        const uint64_t best = wave_max_key((static_cast<uint64_t>(bh) << 32) | static_cast<uint32_t>(~bi));
        bh = static_cast<uint32_t>(best >> 32);
        bi = ~static_cast<uint32_t>(best);
        float bv;
        if (bh == 0) {
            // No candidate left (all remaining -inf): rank keeps -inf with
            // id 0, as the insertion scan leaves it.
            bv = -INFINITY;
            bi = 0;
        } else {
            bv = __uint_as_float(bh - 1u);
            if ((bi & 63u) == lane) {
#pragma unroll
                for (uint32_t r = 0; r < PL; ++r) {
                    if (r == (bi >> 6)) key_hi[r] = 0;
                }
            }
        }
        if (lane == rank) {
            my_v = bv;
            my_i = bi;
        }
    }
    const float sum = wave_sum(lane < k ? my_v : 0.0f);
    if (lane < k) {
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        ids[lane] = static_cast<int32_t>(my_i);
        weights[lane] = my_v * inv;
    }
}

}  // namespace hipllm
