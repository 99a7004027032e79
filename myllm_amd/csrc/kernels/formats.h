// Bit-exact element dequantization of the GGUF block formats (device side).
//
// Restates the reference dequantizers (model.cpp:581-683) element by element,
// with the same operand order and no contraction into FMA, so every value is
// bit-identical to CPULLM's FP32 weights:
//   Q4_K  v = (d * sc) * q - (dmin * m)          model.cpp:630-640
//   Q6_K  v = (d * sc) * (q - 32)                model.cpp:669-676
//   Q8_0  v = q * d                              model.cpp:610-612
//   Q5_0  v = q * d - 16 * d                     model.cpp:595-598
//   F16   exact half_to_float                    model.cpp:500-522
// Byte loads only, so any row alignment works.
#pragma once

#include "common.h"

namespace hipllm {

__device__ inline float dequant_element(uint32_t type, const uint8_t* row, uint32_t col) {
#pragma clang fp contract(off)
    switch (type) {
    case kF32: {
        const uint32_t b = row[4 * col] | (row[4 * col + 1] << 8) | (row[4 * col + 2] << 16) |
                           (static_cast<uint32_t>(row[4 * col + 3]) << 24);
        return __uint_as_float(b);
    }
    case kF16:
        return half_bits_to_float_exact(row[2 * col] | (row[2 * col + 1] << 8));
    case kQ8_0: {
        const uint8_t* blk = row + (col / 32) * 34;
        const float d = half_bits_to_float_exact(blk[0] | (blk[1] << 8));
        const int8_t q = static_cast<int8_t>(blk[2 + col % 32]);
        return static_cast<float>(q) * d;
    }
    case kQ5_0: {
        const uint8_t* blk = row + (col / 32) * 22;
        const float d = half_bits_to_float_exact(blk[0] | (blk[1] << 8));
        const uint32_t qh = blk[2] | (blk[3] << 8) | (blk[4] << 16) | (static_cast<uint32_t>(blk[5]) << 24);
        const uint32_t i = col % 32;
        const uint32_t j = i & 15;
        int q;
        if (i < 16) {
            q = (blk[6 + j] & 0x0f) | static_cast<int>(((qh >> j) << 4) & 0x10);
        } else {
            q = (blk[6 + j] >> 4) | static_cast<int>((qh >> (j + 12)) & 0x10);
        }
        const float a = static_cast<float>(q) * d;
        const float b = 16.0f * d;
        return a - b;
    }
    case kQ4_K: {
        const uint8_t* blk = row + (col / 256) * 144;
        const float d = half_bits_to_float_exact(blk[0] | (blk[1] << 8));
        const float dmin = half_bits_to_float_exact(blk[2] | (blk[3] << 8));
        const uint8_t* s = blk + 4;
        const uint32_t i = col % 256;
        const uint32_t group = i / 64;       // 64-element group, two sub-blocks
        const uint32_t within = i % 64;
        const uint32_t sub = group * 2 + (within >= 32 ? 1 : 0);
        uint32_t sc, m;
        if (sub < 4) {
            sc = s[sub] & 63;
            m = s[sub + 4] & 63;
        } else {
            sc = (s[sub + 4] & 0x0f) | ((s[sub - 4] >> 6) << 4);
            m = (s[sub + 4] >> 4) | ((s[sub] >> 6) << 4);
        }
        const uint8_t qb = blk[16 + group * 32 + (within & 31)];
        const uint32_t q = within < 32 ? (qb & 0x0f) : (qb >> 4);
        const float d1 = d * static_cast<float>(sc);
        const float m1 = dmin * static_cast<float>(m);
        const float t = d1 * static_cast<float>(q);
        return t - m1;
    }
    case kQ6_K: {
        const uint8_t* blk = row + (col / 256) * 210;
        const uint32_t i = col % 256;
        const uint32_t n = i / 128;           // half
        const uint32_t r = i % 128;
        const uint32_t quarter = r / 32;      // 0..3 -> q1..q4
        const uint32_t l = r % 32;
        const uint8_t* ql = blk + 64 * n;
        const uint8_t* qh = blk + 128 + 32 * n;
        const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192);
        const float d = half_bits_to_float_exact(blk[208] | (blk[209] << 8));
        const uint32_t lowbyte = ql[l + (quarter & 1) * 32];
        const uint32_t low = quarter < 2 ? (lowbyte & 0x0f) : (lowbyte >> 4);
        const uint32_t high = (qh[l] >> (2 * quarter)) & 3;
        const int q = static_cast<int>(low | (high << 4)) - 32;
        const int scale = sc[8 * n + l / 16 + 2 * quarter];
        const float ds = d * static_cast<float>(scale);
        return ds * static_cast<float>(q);
    }
    default:
        return 0.0f;
    }
}

}  // namespace hipllm
