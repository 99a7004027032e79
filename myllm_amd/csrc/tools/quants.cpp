// GGML block quantizers (restated from the published ggml reference
// algorithms) and the deterministic random source for synthetic inputs.
#include "quants.h"

#include <cmath>
#include <cstring>
#include <algorithm>

namespace hipllm_tools {

namespace {

constexpr float kGroupMaxEps = 1e-15f;

// Round to nearest, ties to even, through the 1.5 * 2^23 magic constant, as
// ggml's nearest_int does. Valid for |value| <= 2^22.
inline int nearest_int(float value) {
    float shifted = value + 12582912.0f;
    int bits;
    std::memcpy(&bits, &shifted, sizeof(bits));
    return (bits & 0x007fffff) - 0x00400000;
}

inline void store_u16(uint8_t* dst, uint16_t v) {
    dst[0] = static_cast<uint8_t>(v & 0xff);
    dst[1] = static_cast<uint8_t>(v >> 8);
}

// Asymmetric (scale, min) fit for one group, ggml's make_qkx2_quants.
float make_qkx2_quants(int n, int nmax, const float* x, const float* weights,
                       uint8_t* L, float* the_min, uint8_t* Laux, float rmin,
                       float rdelta, int nstep, bool use_mad) {
    float min = x[0];
    float max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.0f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        L[i] = static_cast<uint8_t>(std::max(0, std::min(nmax, l)));
        float diff = scale * L[i] + min - x[i];
        diff = use_mad ? std::fabs(diff) : diff * diff;
        best_error += weights[i] * diff;
    }
    if (nstep < 1) {
        *the_min = -min;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = std::max(0, std::min(nmax, l));
            Laux[i] = static_cast<uint8_t>(l);
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = use_mad ? std::fabs(diff) : diff * diff;
                cur_error += weights[i] * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

// Symmetric scale search, ggml's make_qx_quants with rmse_type = 1
// (weights x^2). L receives values offset by nmax.
float make_qx_quants_rmse1(int n, int nmax, const float* x, int8_t* L) {
    float max = 0;
    float amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = std::fabs(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < kGroupMaxEps) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = -nmax / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = std::max(-nmax, std::min(nmax - 1, l));
        L[i] = static_cast<int8_t>(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = std::max(-nmax, std::min(nmax - 1, l));
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                L[i] = static_cast<int8_t>(nmax + std::max(-nmax, std::min(nmax - 1, l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

// Q8_0: 32 values, f16 scale d = amax/127, int8 quants.
void quantize_q8_0(const float* x, size_t cols, uint8_t* y) {
    for (size_t b = 0; b < cols / 32; ++b) {
        const float* xb = x + b * 32;
        uint8_t* yb = y + b * 34;
        float amax = 0;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(xb[j]));
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        store_u16(yb, float_to_half(d));
        for (int j = 0; j < 32; ++j) {
            const float v = xb[j] * id;
            yb[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(std::roundf(v)));
        }
    }
}

// Q5_0: 32 values, f16 scale d = max/-16, 5-bit quants split in nibbles +
// a 32-bit high-bit mask.
void quantize_q5_0(const float* x, size_t cols, uint8_t* y) {
    for (size_t b = 0; b < cols / 32; ++b) {
        const float* xb = x + b * 32;
        uint8_t* yb = y + b * 22;
        float amax = 0, max = 0;
        for (int j = 0; j < 32; ++j) {
            const float v = xb[j];
            if (amax < std::fabs(v)) {
                amax = std::fabs(v);
                max = v;
            }
        }
        const float d = max / -16;
        const float id = d ? 1.0f / d : 0.0f;
        store_u16(yb, float_to_half(d));
        uint32_t qh = 0;
        uint8_t* qs = yb + 6;
        for (int j = 0; j < 16; ++j) {
            const float x0 = xb[j] * id;
            const float x1 = xb[16 + j] * id;
            const uint8_t xi0 = static_cast<uint8_t>(std::min<int>(31, static_cast<int8_t>(x0 + 16.5f)));
            const uint8_t xi1 = static_cast<uint8_t>(std::min<int>(31, static_cast<int8_t>(x1 + 16.5f)));
            qs[j] = static_cast<uint8_t>((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
            qh |= ((xi0 & 0x10u) >> 4) << (j + 0);
            qh |= ((xi1 & 0x10u) >> 4) << (j + 16);
        }
        yb[2] = static_cast<uint8_t>(qh & 0xff);
        yb[3] = static_cast<uint8_t>((qh >> 8) & 0xff);
        yb[4] = static_cast<uint8_t>((qh >> 16) & 0xff);
        yb[5] = static_cast<uint8_t>((qh >> 24) & 0xff);
    }
}

void get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = static_cast<uint8_t>((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = static_cast<uint8_t>((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

// Q4_K: 256-value super-block = 8 groups of 32 with 6-bit scales/mins
// relative to f16 d/dmin. Layout: d, dmin, scales[12], qs[128].
void quantize_q4_k(const float* x, size_t cols, uint8_t* y) {
    uint8_t L[256];
    uint8_t Laux[32];
    float weights[32];
    float mins[8];
    float scales[8];
    for (size_t b = 0; b < cols / 256; ++b) {
        const float* xb = x + b * 256;
        uint8_t* yb = y + b * 144;
        uint8_t* ys = yb + 4;
        uint8_t* yq = yb + 16;
        std::memset(yb, 0, 144);
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += xb[32 * j + l] * xb[32 * j + l];
            const float av_x = std::sqrt(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + std::fabs(xb[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 15, xb + 32 * j, weights, L + 32 * j,
                                         &mins[j], Laux, -1.0f, 0.1f, 20, false);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
        const float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
        for (int j = 0; j < 8; ++j) {
            uint8_t ls = static_cast<uint8_t>(std::min(63, nearest_int(inv_scale * scales[j])));
            uint8_t lm = static_cast<uint8_t>(std::min(63, nearest_int(inv_min * mins[j])));
            if (j < 4) {
                ys[j] = ls;
                ys[j + 4] = lm;
            } else {
                ys[j + 4] = static_cast<uint8_t>((ls & 0xF) | ((lm & 0xF) << 4));
                ys[j - 4] |= static_cast<uint8_t>((ls >> 4) << 6);
                ys[j - 0] |= static_cast<uint8_t>((lm >> 4) << 6);
            }
        }
        const uint16_t dh = float_to_half(max_scale / 63.0f);
        const uint16_t mh = float_to_half(max_min / 63.0f);
        store_u16(yb, dh);
        store_u16(yb + 2, mh);
        const float dd = half_to_float(dh);
        const float dm_all = half_to_float(mh);
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            get_scale_min_k4(j, ys, &sc, &m);
            const float d = dd * sc;
            if (!d) continue;
            const float dm = dm_all * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((xb[32 * j + ii] + dm) / d);
                l = std::max(0, std::min(15, l));
                L[32 * j + ii] = static_cast<uint8_t>(l);
            }
        }
        uint8_t* q = yq;
        for (int j = 0; j < 256; j += 64) {
            for (int l = 0; l < 32; ++l) {
                q[l] = static_cast<uint8_t>(L[j + l] | (L[j + l + 32] << 4));
            }
            q += 32;
        }
    }
}

// Q6_K: 256-value super-block = 16 groups of 16 with int8 scales relative to
// an f16 d. Layout: ql[128], qh[64], scales[16], d.
void quantize_q6_k(const float* x, size_t cols, uint8_t* y) {
    int8_t L[256];
    float scales[16];
    for (size_t b = 0; b < cols / 256; ++b) {
        const float* xb = x + b * 256;
        uint8_t* yb = y + b * 210;
        std::memset(yb, 0, 210);
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < 16; ++ib) {
            const float scale = make_qx_quants_rmse1(16, 32, xb + 16 * ib, L + 16 * ib);
            scales[ib] = scale;
            const float abs_scale = std::fabs(scale);
            if (abs_scale > max_abs_scale) {
                max_abs_scale = abs_scale;
                max_scale = scale;
            }
        }
        if (max_abs_scale < kGroupMaxEps) {
            store_u16(yb + 208, float_to_half(0.0f));
            continue;
        }
        const float iscale = -128.0f / max_scale;
        const uint16_t dh = float_to_half(1 / iscale);
        store_u16(yb + 208, dh);
        int8_t* ysc = reinterpret_cast<int8_t*>(yb + 192);
        for (int ib = 0; ib < 16; ++ib) {
            ysc[ib] = static_cast<int8_t>(std::min(127, nearest_int(iscale * scales[ib])));
        }
        const float dd = half_to_float(dh);
        for (int j = 0; j < 16; ++j) {
            const float d = dd * ysc[j];
            if (!d) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(xb[16 * j + ii] / d);
                l = std::max(-32, std::min(31, l));
                L[16 * j + ii] = static_cast<int8_t>(l + 32);
            }
        }
        uint8_t* ql = yb;
        uint8_t* qh = yb + 128;
        for (int j = 0; j < 256; j += 128) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = L[j + l + 0] & 0xF;
                const uint8_t q2 = L[j + l + 32] & 0xF;
                const uint8_t q3 = L[j + l + 64] & 0xF;
                const uint8_t q4 = L[j + l + 96] & 0xF;
                ql[l + 0] = static_cast<uint8_t>(q1 | (q3 << 4));
                ql[l + 32] = static_cast<uint8_t>(q2 | (q4 << 4));
                qh[l] = static_cast<uint8_t>((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) |
                                             ((L[j + l + 64] >> 4) << 4) |
                                             ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
    }
}

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

inline uint64_t hash3(uint64_t seed, uint64_t stream, uint64_t index) {
    return mix64(mix64(mix64(seed + 0x9e3779b97f4a7c15ULL) ^ stream) + index * 0x9e3779b97f4a7c15ULL);
}

}  // namespace

uint16_t float_to_half(float value) {
    uint32_t bits;
    std::memcpy(&bits, &value, sizeof(bits));
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t exponent = (bits >> 23) & 0xffu;
    uint32_t mantissa = bits & 0x7fffffu;
    if (exponent == 0xff) {
        return static_cast<uint16_t>(sign | 0x7c00u | (mantissa ? 0x200u : 0u));
    }
    const int e = static_cast<int>(exponent) - 127 + 15;
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return static_cast<uint16_t>(sign);
        mantissa |= 0x800000u;
        const int shift = 14 - e;
        uint32_t half_m = mantissa >> shift;
        const uint32_t rem = mantissa & ((1u << shift) - 1);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_m & 1u))) ++half_m;
        return static_cast<uint16_t>(sign | half_m);
    }
    uint32_t half = sign | (static_cast<uint32_t>(e) << 10) | (mantissa >> 13);
    const uint32_t rem = mantissa & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) ++half;
    return static_cast<uint16_t>(half);
}

float half_to_float(uint16_t value) {
    const uint32_t sign = static_cast<uint32_t>(value >> 15);
    const uint32_t exponent = (value >> 10) & 0x1f;
    const uint32_t mantissa = value & 0x3ff;
    float result;
    if (exponent == 0) {
        result = std::ldexp(static_cast<float>(mantissa) / 1024.0f, -14);
    } else if (exponent == 31) {
        result = mantissa ? NAN : INFINITY;
    } else {
        result = std::ldexp(1.0f + static_cast<float>(mantissa) / 1024.0f,
                            static_cast<int>(exponent) - 15);
    }
    return sign ? -result : result;
}

size_t row_bytes(uint32_t type, size_t cols) {
    switch (type) {
    case kTypeF32: return cols * 4;
    case kTypeF16: return cols * 2;
    case kTypeQ5_0: return cols % 32 ? 0 : cols / 32 * 22;
    case kTypeQ8_0: return cols % 32 ? 0 : cols / 32 * 34;
    case kTypeQ4_K: return cols % 256 ? 0 : cols / 256 * 144;
    case kTypeQ6_K: return cols % 256 ? 0 : cols / 256 * 210;
    default: return 0;
    }
}

bool quantize_row(uint32_t type, const float* src, size_t cols, uint8_t* dst) {
    if (row_bytes(type, cols) == 0 && cols != 0) return false;
    switch (type) {
    case kTypeF32:
        std::memcpy(dst, src, cols * 4);
        return true;
    case kTypeF16:
        for (size_t i = 0; i < cols; ++i) store_u16(dst + 2 * i, float_to_half(src[i]));
        return true;
    case kTypeQ5_0: quantize_q5_0(src, cols, dst); return true;
    case kTypeQ8_0: quantize_q8_0(src, cols, dst); return true;
    case kTypeQ4_K: quantize_q4_k(src, cols, dst); return true;
    case kTypeQ6_K: quantize_q6_k(src, cols, dst); return true;
    default: return false;
    }
}

void fill_normal(uint64_t seed, uint64_t stream, uint64_t first, size_t count,
                 float stddev, float* dst) {
    // Element i takes the cosine (even i) or sine (odd i) branch of the
    // Box-Muller pair number i / 2.
    for (size_t n = 0; n < count; ++n) {
        const uint64_t i = first + n;
        const uint64_t pair = i >> 1;
        const uint64_t h1 = hash3(seed, stream, 2 * pair);
        const uint64_t h2 = hash3(seed, stream, 2 * pair + 1);
        const double u1 = (static_cast<double>(h1 >> 11) + 1.0) * (1.0 / 9007199254740993.0);
        const double u2 = static_cast<double>(h2 >> 11) * (1.0 / 9007199254740992.0);
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double angle = 6.283185307179586 * u2;
        const double z = (i & 1) ? r * std::sin(angle) : r * std::cos(angle);
        dst[n] = static_cast<float>(z * stddev);
    }
}

void fill_uniform_int(uint64_t seed, uint64_t stream, uint64_t first,
                      size_t count, uint32_t bound, int32_t* dst) {
    for (size_t n = 0; n < count; ++n) {
        const uint64_t h = hash3(seed, stream, first + n);
        dst[n] = static_cast<int32_t>((h >> 32) * bound >> 32);
    }
}

}  // namespace hipllm_tools
