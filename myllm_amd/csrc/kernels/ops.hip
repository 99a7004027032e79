// Decode-path operators around the GEMV: RMSNorm, embedding gather, RoPE +
// KV-cache write, GQA attention over the device KV cache, argmax.
//
// Reference semantics (file:line):
//   RMSNorm      cpu_llm.cpp:143-166 (double sum of squares; x *= inv * g)
//   embedding    cpu_llm.cpp:101-123, metal_llm.metal:1066-1162
//   RoPE (NeoX)  cpu_llm.cpp:204-235; K is cached after rotation (874-886)
//   attention    cpu_llm.cpp:490-510 (scores * (1/sqrt(D))), 168-186 (softmax),
//                453-467 (p . V); GQA head map h / (Hq / Hkv) (897-905)
//   argmax       cpu_llm.cpp:34-48 (first maximum), metal_llm.metal:1544-1644
#include "formats.h"
#include "norm.h"
#include "router.h"

namespace hipllm {
namespace {

// ------------------------------------------------------------ RMSNorm
// One block per row (norm.h): y and, optionally, its XGroup form for the GEMV
// that consumes it.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                      float* __restrict__ y, XGroup* __restrict__ yq, uint32_t cols,
                                                      float eps) {
    const size_t row = blockIdx.x;
    rmsnorm_row(x + row * cols, gamma, y + row * cols, yq ? yq + row * (cols / 16) : nullptr, cols, eps);
}

// ------------------------------------------------------------ embedding

__global__ void embed_kernel(uint32_t type, const uint8_t* __restrict__ table, size_t row_bytes,
                             const int32_t* __restrict__ ids, uint32_t vocab, uint32_t cols,
                             float* __restrict__ out) {
    const uint32_t t = blockIdx.y;
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= cols) return;
    const int32_t id = ids[t];
    float v = 0.0f;
    if (id >= 0 && static_cast<uint32_t>(id) < vocab) {
        v = dequant_element(type, table + static_cast<size_t>(id) * row_bytes, c);
    }
    out[static_cast<size_t>(t) * cols + c] = v;
}

// ------------------------------------------------------------ RoPE + KV
// qkv rows hold [Q (Hq*D) | K (Hkv*D) | V (Hkv*D)] with biases applied. Row r
// is at absolute position pos0 + r. Rotates Q and K in place with the
// host-built table (cos, sin per position and pair, computed exactly as
// CPULLM computes them), stores rotated K and V into the caches at row
// pos0 + r, and leaves rotated Q in place.
#pragma clang fp contract(off)
// Element i of a head rotated with the position's (cos, sin) pairs, the same
// products and sum as rope_kv_kernel (contraction off): pairs (p, p + half)
// for p < half, dims past 2 half unchanged.
// Element i of the rotated row x, cs = the table pair of i (of i - half in
// the second half; unused past 2 half).
__device__ __forceinline__ float rope_apply(const float* __restrict__ x, float2 cs, uint32_t half, uint32_t i) {
    if (i < half) {
        const float t1 = x[i] * cs.x;
        const float t2 = x[i + half] * cs.y;
        return t1 - t2;
    }
    if (i < 2 * half) {
        const float t3 = x[i - half] * cs.y;
        const float t4 = x[i] * cs.x;
        return t3 + t4;
    }
    return x[i];
}

__device__ __forceinline__ float rope_elem(const float* __restrict__ x, const float2* __restrict__ tab, uint32_t half,
                                          uint32_t i) {
    const float2 cs = i < 2 * half ? tab[i < half ? i : i - half] : make_float2(0.0f, 0.0f);
    return rope_apply(x, cs, half, i);
}

__global__ void rope_kv_kernel(float* __restrict__ qkv, const float2* __restrict__ table, uint32_t half_rot,
                               uint32_t hq, uint32_t hkv, uint32_t d, uint32_t pos0, uint32_t row_stride,
                               float* __restrict__ kcache, float* __restrict__ vcache,
                               const uint32_t* __restrict__ dpos) {
    const uint32_t r = blockIdx.x;
    float* row = qkv + static_cast<size_t>(r) * row_stride;
    const uint32_t pos = (dpos ? *dpos : pos0) + r;
    const uint32_t kvd = hkv * d;
    const float2* tab = table + static_cast<size_t>(pos) * half_rot;
    const uint32_t heads = hq + hkv;
    const uint32_t half = d / 2;
    for (uint32_t i = threadIdx.x; i < heads * half; i += blockDim.x) {
        const uint32_t h = i / half;
        const uint32_t p = i % half;
        float* base = row + h * d;  // Q heads then K heads are contiguous
        if (p < half_rot) {
            const float2 cs = tab[p];
            const float a = base[p];
            const float b = base[p + half_rot];
            const float t1 = a * cs.x;
            const float t2 = b * cs.y;
            const float t3 = a * cs.y;
            const float t4 = b * cs.x;
            base[p] = t1 - t2;
            base[p + half_rot] = t3 + t4;
        }
    }
    __syncthreads();
    float* kc = kcache + static_cast<size_t>(pos) * kvd;
    float* vc = vcache + static_cast<size_t>(pos) * kvd;
    for (uint32_t i = threadIdx.x; i < kvd; i += blockDim.x) {
        kc[i] = row[hq * d + i];
        vc[i] = row[hq * d + kvd + i];
    }
}
#pragma clang fp contract(fast)

// ------------------------------------------------------------ attention
// Split-K decode attention (flash-decode). Phase 1: block (head, split y)
// processes the 64-key chunks y, y + S, y + 2S, ... of [0, len) (S splits):
// per chunk, four lanes per key score it against the query (each a quarter of
// the head dims), then p.V accumulates in registers (threads split the
// chunk's keys in 256 / (D / 4) interleaved parts), with an online softmax
// across the block's chunks. It writes its running max m, sum of exp l and
// unnormalised p.V (D floats; m = -inf, l = 0 for a split without keys).
// Phase 2: one block per head merges the S splits and writes the head output,
// plus its XGroup form for the next GEMV. The length is a value or, for
// launches recorded once and replayed per token, read from device memory
// (len = *dpos + 1); S then follows the capacity, not the length.
constexpr uint32_t kAttnChunk = 64;
constexpr uint32_t kAttnMaxSplits = 16;
constexpr uint32_t kAttnHeadChunks = 4;  // up to 4 split-sized chunks merged inside one block

// With rope != nullptr (the fused decode step), q is this token's raw qkv row
// ([Q heads | K heads | V heads]): the block rotates its query head into LDS,
// and the block(s) whose split holds the token's own key (the last chunk)
// rotate that key head, write it and the value head into the caches at row
// len - 1, then synchronise before reading them. Every head of a KV group
// writes the same values there, so the duplicate writes agree.
//
// With one split (short capacities) the block finishes the head itself: out,
// outq (nullable) and the optional sigmoid gate exactly as the merge computes
// them for a single split (weight exp(0) = 1), so no merge launch follows.
//
// DT (64 or 128; 0 = any d, given at run time): the block's first chunk has
// its K and V rows loaded at the start, before the RoPE and the barrier, so
// a split with one chunk waits for one memory round trip; its token's own
// row, written by this launch, comes from the block's rotated values.
template <uint32_t DT>
__global__ __launch_bounds__(256) void attn_decode_partial(const float* __restrict__ q, float* __restrict__ kcache,
                                                           float* __restrict__ vcache, float* __restrict__ part,
                                                           uint32_t hq, uint32_t hkv, uint32_t d_arg, uint32_t len_arg,
                                                           const uint32_t* __restrict__ dpos, float scale,
                                                           uint32_t splits, const float2* __restrict__ rope,
                                                           uint32_t half_rot, float* __restrict__ fout,
                                                           XGroup* __restrict__ foutq,
                                                           const float* __restrict__ gate) {
    constexpr bool kPre = DT != 0;
    constexpr uint32_t KR = kPre ? DT / 16 : 1;          // float4 of a key per scoring lane
    constexpr uint32_t VR = kPre ? kAttnChunk * DT / 1024 : 1;  // value rows per p.V lane
    const uint32_t d = kPre ? DT : d_arg;
    const uint32_t h = blockIdx.x;
    const uint32_t split = blockIdx.y;
    const uint32_t len = dpos ? *dpos + 1 : len_arg;
    const uint32_t nchunks = (len + kAttnChunk - 1) / kAttnChunk;
    const uint32_t g = h / (hq / hkv);
    const uint32_t kvd = hkv * d;
    __shared__ float4 qs4[64];
    __shared__ float4 kn4[kPre ? DT / 4 : 1], vn4[kPre ? DT / 4 : 1];
    __shared__ float ps[kAttnChunk];
    __shared__ float red[8];
    __shared__ float4 accp[256];
    const uint32_t tid = threadIdx.x;
    const uint32_t d4 = d / 4;
    const uint32_t wave = tid >> 6, lane = tid & 63;
    // p.V ownership: float4 column c4 = tid % (d / 4), key subset pp = tid /
    // (d / 4) of `parts` (threads past parts * d / 4 idle).
    const uint32_t parts = blockDim.x / d4;
    const bool pv = tid < parts * d4;
    const uint32_t c4 = tid % d4, pp = tid / d4;
    // Scores: key j = tid / 4, quarter qq = tid % 4 covers float4 columns qq, qq + 4, ...
    const uint32_t j = tid >> 2, qq = tid & 3;
    const uint32_t newrow = rope ? len - 1 : 0xffffffffu;
    float4 kr[KR], vr[VR];
    if constexpr (kPre) {
        if (split < nchunks) {
            const uint32_t t0 = split * kAttnChunk;
            const uint32_t cnt = min(len - t0, kAttnChunk);
            if (j < cnt && t0 + j != newrow) {
                const float4* k = reinterpret_cast<const float4*>(kcache + static_cast<size_t>(t0 + j) * kvd + g * d);
#pragma unroll
                for (uint32_t r = 0; r < KR; ++r) kr[r] = k[qq + 4 * r];
            }
            const float4* v = reinterpret_cast<const float4*>(vcache + static_cast<size_t>(t0) * kvd + g * d) + c4;
#pragma unroll
            for (uint32_t r = 0; r < VR; ++r) {
                const uint32_t jj = pp + r * (256 / (DT / 4));
                if (jj < cnt && t0 + jj != newrow) vr[r] = v[static_cast<size_t>(jj) * (kvd / 4)];
            }
        }
    }
    if (rope) {
        const float2* tab = rope + static_cast<size_t>(len - 1) * half_rot;
        float* qs = reinterpret_cast<float*>(qs4);
        for (uint32_t i = tid; i < d; i += blockDim.x) qs[i] = rope_elem(q + h * d, tab, half_rot, i);
        if ((nchunks - 1) % splits == split) {
            const float* kn = q + hq * d + g * d;
            const float* vn = kn + kvd;
            float* kc = kcache + static_cast<size_t>(len - 1) * kvd + g * d;
            float* vc = vcache + static_cast<size_t>(len - 1) * kvd + g * d;
            for (uint32_t i = tid; i < d; i += blockDim.x) {
                const float kv = rope_elem(kn, tab, half_rot, i);
                kc[i] = kv;
                vc[i] = vn[i];
                if constexpr (kPre) {
                    reinterpret_cast<float*>(kn4)[i] = kv;
                    reinterpret_cast<float*>(vn4)[i] = vn[i];
                }
            }
        }
    } else {
        for (uint32_t i = tid; i < d4; i += blockDim.x) qs4[i] = reinterpret_cast<const float4*>(q + h * d)[i];
    }
    __syncthreads();
    float m_run = -INFINITY, l_run = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t chunk = split; chunk < nchunks; chunk += splits) {
        const uint32_t t0 = chunk * kAttnChunk;
        const uint32_t cnt = min(len - t0, kAttnChunk);
        const bool first = kPre && chunk == split;  // rows held in registers
        float s = -INFINITY;
        {
            float dot = 0.0f;
            if (j < cnt) {
                const float4* k = reinterpret_cast<const float4*>(kcache + static_cast<size_t>(t0 + j) * kvd + g * d);
                const bool own = t0 + j == newrow;
                if (first) {
#pragma unroll
                    for (uint32_t r = 0; r < KR; ++r) {
                        const float4 kv = own ? kn4[qq + 4 * r] : kr[r];
                        const float4 qv = qs4[qq + 4 * r];
                        dot = fmaf(kv.x, qv.x, dot);
                        dot = fmaf(kv.y, qv.y, dot);
                        dot = fmaf(kv.z, qv.z, dot);
                        dot = fmaf(kv.w, qv.w, dot);
                    }
                } else {
                    for (uint32_t i = qq; i < d4; i += 4) {
                        const float4 kv = k[i];
                        const float4 qv = qs4[i];
                        dot = fmaf(kv.x, qv.x, dot);
                        dot = fmaf(kv.y, qv.y, dot);
                        dot = fmaf(kv.z, qv.z, dot);
                        dot = fmaf(kv.w, qv.w, dot);
                    }
                }
            }
            dot = quad_sum(dot);
            if (j < cnt) s = dot * scale;
        }
        float cm = wave_max(s);
        if (lane == 0) red[wave] = cm;
        __syncthreads();
        cm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        const float m_new = fmaxf(m_run, cm);  // finite: every chunk holds a key
        const float p = j < cnt ? expf(s - m_new) : 0.0f;
        if (qq == 0) ps[j] = p;
        float l = wave_sum(qq == 0 ? p : 0.0f);
        __syncthreads();  // red[0..3] read by all; ps[] complete
        if (lane == 0) red[4 + wave] = l;
        __syncthreads();
        l = (red[4] + red[5]) + (red[6] + red[7]);
        const float corr = expf(m_run - m_new);  // 0 on the first chunk
        l_run = l_run * corr + l;
        m_run = m_new;
        if (pv) {
            const float4* v = reinterpret_cast<const float4*>(vcache + static_cast<size_t>(t0) * kvd + g * d) + c4;
            float4 a = make_float4(acc.x * corr, acc.y * corr, acc.z * corr, acc.w * corr);
            if (first) {
#pragma unroll
                for (uint32_t r = 0; r < VR; ++r) {
                    const uint32_t jj = pp + r * parts;
                    if (jj < cnt) {
                        const float pj = ps[jj];
                        const float4 vv = t0 + jj == newrow ? vn4[c4] : vr[r];
                        a.x = fmaf(pj, vv.x, a.x);
                        a.y = fmaf(pj, vv.y, a.y);
                        a.z = fmaf(pj, vv.z, a.z);
                        a.w = fmaf(pj, vv.w, a.w);
                    }
                }
            } else {
#pragma unroll 4
                for (uint32_t jj = pp; jj < cnt; jj += parts) {
                    const float pj = ps[jj];
                    const float4 vv = v[static_cast<size_t>(jj) * (kvd / 4)];
                    a.x = fmaf(pj, vv.x, a.x);
                    a.y = fmaf(pj, vv.y, a.y);
                    a.z = fmaf(pj, vv.z, a.z);
                    a.w = fmaf(pj, vv.w, a.w);
                }
            }
            acc = a;
        }
        __syncthreads();  // ps[] and red[] are rewritten by the next chunk
    }
    if (pv) accp[tid] = acc;
    __syncthreads();
    if (splits == 1) {
        __shared__ __align__(16) float vals[256];
        const float invL = 1.0f / l_run;
        for (uint32_t cc = tid; cc < d4; cc += blockDim.x) {
            float4 a = accp[cc];
            for (uint32_t k = 1; k < parts; ++k) {
                const float4 b = accp[k * d4 + cc];
                a.x += b.x;
                a.y += b.y;
                a.z += b.z;
                a.w += b.w;
            }
            const float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const uint32_t i = 4 * cc + j;
                float v = av[j] * invL;
                if (gate) v = v * sigmoid_ref(gate[h * d + i]);
                fout[h * d + i] = v;
                vals[i] = v;
            }
        }
        if (foutq) {
            __syncthreads();
            for (uint32_t gI = tid; gI < d / 16; gI += blockDim.x) {
                xgroup_encode_from(vals + 16 * gI, foutq + h * (d / 16) + gI);
            }
        }
        return;
    }
    float* out = part + (static_cast<size_t>(h) * splits + split) * (d + 2);
    for (uint32_t cc = tid; cc < d4; cc += blockDim.x) {
        float4 a = accp[cc];
        for (uint32_t k = 1; k < parts; ++k) {
            const float4 b = accp[k * d4 + cc];
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
        }
        out[2 + 4 * cc + 0] = a.x;
        out[2 + 4 * cc + 1] = a.y;
        out[2 + 4 * cc + 2] = a.z;
        out[2 + 4 * cc + 3] = a.w;
    }
    if (tid == 0) {
        out[0] = m_run;
        out[1] = l_run;
    }
}

// The split kernel and the merge in one launch for capacities of 2 to NG
// chunks and heads of D = 64, 128 or 256 dims: one block of NG x 256 threads per
// head, thread group c (256 threads) doing what split c of a launch with
// one chunk per split does (scores, softmax and p.V over chunk c), then the
// groups' (m, l, p.V) merged in the block in group order as the merge
// kernel merges splits (a group past the last chunk has m = -inf, l = 0,
// weight 0). For D <= 128 every K and V row a thread uses is loaded at the
// start, before the RoPE and the block barrier, so the block waits for one
// memory round trip (D = 256: K after the barrier, then V); the token's own
// row (len - 1 with rope), which this launch writes into the caches, is
// taken from the block's own rotated values instead.
// Same operations in the same order as the two launches: the output bits
// are equal.
// QG (gated attention with head norms, rope set): q is the interleaved
// [Q_h | gate_h] row (2 D per head) and qg.kv the [K | V] row; wave 0
// RMS-normalises Q_h with qg.q_gamma and wave 1 K_g with qg.k_gamma into LDS
// (split_qgate_norm_kernel's sums and products) before the RoPE, and the
// output gate is gate_h.
struct AttnQGate {
    const float* kv;
    const float* q_gamma;
    const float* k_gamma;
    float eps;
};

template <uint32_t NG, uint32_t D, bool QG = false>
__global__ __launch_bounds__(256 * NG) void attn_decode_head(const float* __restrict__ q, float* __restrict__ kcache,
                                                             float* __restrict__ vcache, uint32_t hq, uint32_t hkv,
                                                             uint32_t len_arg, const uint32_t* __restrict__ dpos,
                                                             float scale, const float2* __restrict__ rope,
                                                             uint32_t half_rot, float* __restrict__ fout,
                                                             XGroup* __restrict__ foutq,
                                                             const float* __restrict__ gate,
                                                             const AttnQGate qg = AttnQGate{}) {
    constexpr uint32_t D4 = D / 4;
    constexpr uint32_t PARTS = 256 / D4;           // p.V key subsets
    constexpr uint32_t KR = D4 / 4;                // float4 of a key per scoring lane
    constexpr uint32_t VR = kAttnChunk / PARTS;    // value rows per p.V lane
    // 256-dim heads load their rows where they are used: a lane's K (64
    // floats) held from the start already exceeds the registers of a
    // 1024-thread block (measured: 48 bytes of scratch per lane).
    constexpr bool kPre = D <= 128;
    static_assert(256 * NG >= D, "one thread per head dimension");
    const uint32_t h = blockIdx.x;
    const uint32_t len = dpos ? *dpos + 1 : len_arg;
    const uint32_t nchunks = (len + kAttnChunk - 1) / kAttnChunk;  // <= NG
    const uint32_t g = h / (hq / hkv);
    const uint32_t kvd = hkv * D;
    const uint32_t newrow = rope ? len - 1 : 0xffffffffu;
    __shared__ float4 qs4[D4], kn4[D4], vn4[D4];
    __shared__ float ps[NG][kAttnChunk];
    __shared__ float red[NG][8];
    __shared__ float ml[NG][2];
    __shared__ float4 accp[256 * NG];
    __shared__ __align__(16) float vals[D];
    const uint32_t tid = threadIdx.x;
    const uint32_t grp = tid >> 8, lt = tid & 255;
    const uint32_t wave = lt >> 6, lane = tid & 63;
    const uint32_t t0 = grp * kAttnChunk;
    const uint32_t cnt = grp < nchunks ? min(len - t0, kAttnChunk) : 0u;
    // Scores: key j = lt / 4, quarter qq = lt % 4 covers float4 columns qq, qq + 4, ...
    const uint32_t j = lt >> 2, qq = lt & 3;
    // p.V: float4 column c4, keys pp, pp + PARTS, ...
    const uint32_t c4 = lt % D4, pp = lt / D4;
    float4 kr[kPre ? KR : 1], vr[kPre ? VR : 1];
    const float4* krow = reinterpret_cast<const float4*>(kcache + static_cast<size_t>(t0 + j) * kvd + g * D);
    if constexpr (kPre) {
        if (j < cnt && t0 + j != newrow) {
#pragma unroll
            for (uint32_t r = 0; r < KR; ++r) kr[r] = krow[qq + 4 * r];
        }
    }
    const float4* vrow = reinterpret_cast<const float4*>(vcache + static_cast<size_t>(t0) * kvd + g * D) + c4;
    if constexpr (kPre) {
#pragma unroll
        for (uint32_t r = 0; r < VR; ++r) {
            const uint32_t jj = pp + r * PARTS;
            if (jj < cnt && t0 + jj != newrow) vr[r] = vrow[static_cast<size_t>(jj) * (kvd / 4)];
        }
    }
    const float* qrow = q + h * D;
    if constexpr (QG) qrow = q + static_cast<size_t>(h) * 2 * D;
    const float* grow = QG ? qrow + D : (gate ? gate + h * D : nullptr);
    // The new row's V value, table pair and output gate of this thread's
    // dimension, loaded now.
    const float* vn = QG ? qg.kv + kvd + g * D : q + hq * D + g * D + kvd;
    float2 cs_pre = make_float2(0.0f, 0.0f);
    float v_pre = 0.0f, g_pre = 0.0f;
    if (tid < D) {
        if (rope) {
            const float2* tab = rope + static_cast<size_t>(len - 1) * half_rot;
            if (tid < 2 * half_rot) cs_pre = tab[tid < half_rot ? tid : tid - half_rot];
            v_pre = vn[tid];
        }
        if (grow) g_pre = grow[tid];
    }
    __shared__ float qgn[QG ? 2 : 1][QG ? D : 1];
    if constexpr (QG) {
        if (tid < 128) {
            const uint32_t wv = tid >> 6;
            const float* src = wv == 0 ? qrow : qg.kv + g * D;
            const float* gam = wv == 0 ? qg.q_gamma : qg.k_gamma;
            float ss = 0.0f;
            for (uint32_t i = lane; i < D; i += 64) ss += src[i] * src[i];
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / static_cast<float>(D) + qg.eps);
            for (uint32_t i = lane; i < D; i += 64) qgn[wv][i] = src[i] * inv * gam[i];
        }
        __syncthreads();
    }
    if (rope) {
        const float* kn = QG ? qgn[QG ? 1 : 0] : q + hq * D + g * D;
        const float* qn = QG ? qgn[0] : qrow;
        float* kc = kcache + static_cast<size_t>(len - 1) * kvd + g * D;
        float* vc = vcache + static_cast<size_t>(len - 1) * kvd + g * D;
        float* qs = reinterpret_cast<float*>(qs4);
        float* ks = reinterpret_cast<float*>(kn4);
        float* vs = reinterpret_cast<float*>(vn4);
        if (tid < D) {
            const uint32_t i = tid;
            qs[i] = rope_apply(qn, cs_pre, half_rot, i);
            const float kv = rope_apply(kn, cs_pre, half_rot, i);
            ks[i] = kv;
            vs[i] = v_pre;
            kc[i] = kv;
            vc[i] = v_pre;
        }
    } else {
        for (uint32_t i = tid; i < D4; i += blockDim.x) qs4[i] = reinterpret_cast<const float4*>(q + h * D)[i];
    }
    __syncthreads();
    float s = -INFINITY;
    {
        float dot = 0.0f;
        if (j < cnt) {
            const bool own = t0 + j == newrow;
#pragma unroll
            for (uint32_t r = 0; r < KR; ++r) {
                float4 kv;
                if constexpr (kPre) {
                    kv = own ? kn4[qq + 4 * r] : kr[r];
                } else {
                    kv = own ? kn4[qq + 4 * r] : krow[qq + 4 * r];
                }
                const float4 qv = qs4[qq + 4 * r];
                dot = fmaf(kv.x, qv.x, dot);
                dot = fmaf(kv.y, qv.y, dot);
                dot = fmaf(kv.z, qv.z, dot);
                dot = fmaf(kv.w, qv.w, dot);
            }
        }
        dot = quad_sum(dot);
        if (j < cnt) s = dot * scale;
    }
    float cm = wave_max(s);
    if (lane == 0) red[grp][wave] = cm;
    __syncthreads();
    cm = fmaxf(fmaxf(red[grp][0], red[grp][1]), fmaxf(red[grp][2], red[grp][3]));  // -inf without keys
    const float p = j < cnt ? expf(s - cm) : 0.0f;
    if (qq == 0) ps[grp][j] = p;
    float l = wave_sum(qq == 0 ? p : 0.0f);
    __syncthreads();
    if (lane == 0) red[grp][4 + wave] = l;
    __syncthreads();
    l = (red[grp][4] + red[grp][5]) + (red[grp][6] + red[grp][7]);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (uint32_t r = 0; r < VR; ++r) {
        const uint32_t jj = pp + r * PARTS;
        if (jj < cnt) {
            const float pj = ps[grp][jj];
            float4 vv;
            if constexpr (kPre) {
                vv = t0 + jj == newrow ? vn4[c4] : vr[r];
            } else {
                vv = t0 + jj == newrow ? vn4[c4] : vrow[static_cast<size_t>(jj) * (kvd / 4)];
            }
            acc.x = fmaf(pj, vv.x, acc.x);
            acc.y = fmaf(pj, vv.y, acc.y);
            acc.z = fmaf(pj, vv.z, acc.z);
            acc.w = fmaf(pj, vv.w, acc.w);
        }
    }
    accp[tid] = acc;
    if (lt == 0) {
        ml[grp][0] = cnt ? cm : -INFINITY;
        ml[grp][1] = cnt ? l : 0.0f;
    }
    __syncthreads();
    // Merge: thread i < D owns output dim i, groups in order.
    if (tid < D) {
        const uint32_t cc = tid >> 2, comp = tid & 3;
        float M = -INFINITY;
#pragma unroll
        for (uint32_t c = 0; c < NG; ++c) {
            if (c < nchunks) M = fmaxf(M, ml[c][0]);
        }
        float L = 0.0f, a = 0.0f;
#pragma unroll
        for (uint32_t c = 0; c < NG; ++c) {
            if (c < nchunks) {
                float4 v = accp[c * 256 + cc];
#pragma unroll
                for (uint32_t k = 1; k < PARTS; ++k) {
                    const float4 b = accp[c * 256 + k * D4 + cc];
                    v.x += b.x;
                    v.y += b.y;
                    v.z += b.z;
                    v.w += b.w;
                }
                const float vi = comp == 0 ? v.x : comp == 1 ? v.y : comp == 2 ? v.z : v.w;
                const float wgt = expf(ml[c][0] - M);
                L += ml[c][1] * wgt;
                a += vi * wgt;
            }
        }
        float v = a * (1.0f / L);
        if (grow) v = v * sigmoid_ref(g_pre);
        fout[h * D + tid] = v;
        vals[tid] = v;
    }
    if (foutq) {
        __syncthreads();
        for (uint32_t gI = tid; gI < D / 16; gI += blockDim.x) xgroup_encode_from(vals + 16 * gI, foutq + h * (D / 16) + gI);
    }
}

// gate (nullable): the head outputs are multiplied by sigmoid(gate) (the
// gated attention's output gate, as the separate gate kernel computes it).
// Thread i < d owns output dim i (d <= 256 = blockDim). Every split's m, l
// and value i are loaded at once (one memory round trip; indices past the
// last split repeat it and are not used), then combined in split order.
__global__ __launch_bounds__(256) void attn_decode_merge(const float* __restrict__ part, float* __restrict__ out,
                                                         XGroup* __restrict__ outq, uint32_t d, uint32_t nchunks,
                                                         const float* __restrict__ gate) {
    const uint32_t h = blockIdx.x;
    const uint32_t i = threadIdx.x;
    const float* ph = part + static_cast<size_t>(h) * nchunks * (d + 2);
    // nchunks = the number of splits (<= kAttnMaxSplits); a split without
    // keys has m = -inf, weight exp(-inf - M) = 0 (split 0 always holds key
    // 0, so M is finite).
    const uint32_t ii = min(i, d - 1);
    float ms[kAttnMaxSplits], ls[kAttnMaxSplits], vs[kAttnMaxSplits];
#pragma unroll
    for (uint32_t c = 0; c < kAttnMaxSplits; ++c) {
        const float* pc = ph + static_cast<size_t>(min(c, nchunks - 1)) * (d + 2);
        ms[c] = pc[0];
        ls[c] = pc[1];
        vs[c] = pc[2 + ii];
    }
    float M = -INFINITY;
#pragma unroll
    for (uint32_t c = 0; c < kAttnMaxSplits; ++c) {
        if (c < nchunks) M = fmaxf(M, ms[c]);
    }
    float L = 0.0f, acc = 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < kAttnMaxSplits; ++c) {
        if (c < nchunks) {
            const float wgt = expf(ms[c] - M);
            L += ls[c] * wgt;
            acc += vs[c] * wgt;
        }
    }
    const float invL = 1.0f / L;
    __shared__ __align__(16) float vals[256];
    if (i < d) {
        float v = acc * invL;
        if (gate) v = v * sigmoid_ref(gate[h * d + i]);
        out[h * d + i] = v;
        vals[i] = v;
    }
    __syncthreads();
    if (outq) {
        for (uint32_t gI = threadIdx.x; gI < d / 16; gI += blockDim.x) {
            xgroup_encode_from(vals + 16 * gI, outq + h * (d / 16) + gI);
        }
    }
}

// Causal prefill attention (cpu_llm.cpp:609-629 gemmts + causal_mask
// 316-329 + softmax 168-186 + gemm 549-565; metal_kv_cache_qk/av_f32
// metal_llm.metal:995-1061): block (row r, head h) attends query row r, at
// absolute position pos0 + r, to keys [0, pos0 + r] of the caches. Keys are
// scored 256 at a time (one per thread) with an online softmax; threads
// d < D accumulate the output dimension d, so V rows are read coalesced.
__global__ __launch_bounds__(256) void attn_prefill_kernel(const float* __restrict__ q, uint32_t q_stride,
                                                           const float* __restrict__ kcache,
                                                           const float* __restrict__ vcache, float* __restrict__ out,
                                                           uint32_t out_stride, uint32_t hq, uint32_t hkv, uint32_t d,
                                                           uint32_t pos0, float scale) {
    const uint32_t r = blockIdx.x;
    const uint32_t h = blockIdx.y;
    const uint32_t g = h / (hq / hkv);
    const uint32_t kvd = hkv * d;
    const uint32_t len = pos0 + r + 1;
    __shared__ float qs[256];
    __shared__ float ps[256];
    __shared__ float red[8];
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6, lane = tid & 63;
    for (uint32_t i = tid; i < d; i += blockDim.x) qs[i] = q[static_cast<size_t>(r) * q_stride + h * d + i];
    __syncthreads();
    float m_run = -INFINITY, l_run = 0.0f, acc = 0.0f;
    for (uint32_t t0 = 0; t0 < len; t0 += 256) {
        const uint32_t t = t0 + tid;
        float s = -INFINITY;
        if (t < len) {
            const float4* k = reinterpret_cast<const float4*>(kcache + static_cast<size_t>(t) * kvd + g * d);
            float dot = 0.0f;
            for (uint32_t i = 0; i < d / 4; ++i) {
                const float4 kv = k[i];
                dot = fmaf(kv.x, qs[4 * i], dot);
                dot = fmaf(kv.y, qs[4 * i + 1], dot);
                dot = fmaf(kv.z, qs[4 * i + 2], dot);
                dot = fmaf(kv.w, qs[4 * i + 3], dot);
            }
            s = dot * scale;
        }
        float cm = wave_max(s);
        if (lane == 0) red[wave] = cm;
        __syncthreads();
        cm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        const float m_new = fmaxf(m_run, cm);  // finite: key t0 is always valid
        const float p = t < len ? expf(s - m_new) : 0.0f;
        ps[tid] = p;
        float cs = wave_sum(p);
        __syncthreads();  // red[0..3] read by all before reuse
        if (lane == 0) red[4 + wave] = cs;
        __syncthreads();
        cs = (red[4] + red[5]) + (red[6] + red[7]);
        const float corr = expf(m_run - m_new);
        l_run = l_run * corr + cs;
        if (tid < d) {
            const uint32_t cnt = min(256u, len - t0);
            const float* v = vcache + static_cast<size_t>(t0) * kvd + g * d + tid;
            float a = 0.0f;
            for (uint32_t j = 0; j < cnt; ++j) a = fmaf(ps[j], v[static_cast<size_t>(j) * kvd], a);
            acc = acc * corr + a;
        }
        m_run = m_new;
        __syncthreads();  // ps and red reused by the next chunk
    }
    if (tid < d) out[static_cast<size_t>(r) * out_stride + h * d + tid] = acc / l_run;
}

// The same attention for head size D in {64, 128, 256}, tiled over queries:
// block (tile of QT query rows, head h) keeps the tile's queries in LDS and
// stages K and V KC keys at a time, so each cache row is read from L2 once per
// (tile, head) instead of once per (query row, head). Score phase: thread
// (key j = tid % KC, row group tid / KC) scores RQ rows; the online-softmax
// max and sum run over the KC lanes of a row with xor shuffles. Output phase:
// thread (column x = tid % D, row group tid / D) accumulates RP rows (when the
// tile has fewer scores than threads, row groups past QT idle in the score
// phase). Keys at or past the tile's last position + 1 are staged as zeros,
// so cache rows beyond the prompt are never read. Each chunk's K / V loads
// are issued into registers while the previous chunk is scored.
template <uint32_t D, uint32_t QT>
__global__ __launch_bounds__(256) void attn_prefill_tiled_kernel(const float* __restrict__ q, uint32_t q_stride,
                                                                 const float* __restrict__ kcache,
                                                                 const float* __restrict__ vcache,
                                                                 float* __restrict__ out, uint32_t out_stride,
                                                                 uint32_t rows, uint32_t hq, uint32_t hkv,
                                                                 uint32_t pos0, float scale) {
    constexpr uint32_t KC = 4096 / D;  // keys per chunk
    constexpr uint32_t LDK = D + 4;
    constexpr uint32_t GQ = 256 / KC;  // row groups of the score phase
    constexpr uint32_t RQ = QT > GQ ? QT / GQ : 1;
    constexpr uint32_t RP = QT * D / 256;
    constexpr uint32_t NL = KC * D / 1024;  // float4 of K (and of V) per thread per chunk
    static_assert(KC <= 64 && 64 % KC == 0 && RP >= 1 && QT % RQ == 0 && (QT > GQ ? QT % GQ == 0 : GQ % QT == 0),
                  "tile shape");
    __shared__ __align__(16) float qs[QT * LDK];
    __shared__ __align__(16) float ks[KC * LDK];
    __shared__ __align__(16) float vs[KC * D];
    __shared__ __align__(16) float ps[KC * QT];
    __shared__ float corr[QT];
    __shared__ float lsum[QT];
    const uint32_t tid = threadIdx.x;
    const uint32_t r0 = blockIdx.x * QT, h = blockIdx.y;
    const uint32_t g = h / (hq / hkv);
    const uint32_t kvd = hkv * D;
    const uint32_t nrow = min(QT, rows - r0);
    const uint32_t kend = pos0 + r0 + nrow;  // keys [0, kend) cover every row of the tile
    const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t e = tid; e < QT * D / 4; e += 256) {
        const uint32_t i = e / (D / 4), c = e % (D / 4);
        float4 v = zero4;
        if (i < nrow) v = *reinterpret_cast<const float4*>(q + static_cast<size_t>(r0 + i) * q_stride + h * D + 4 * c);
        *reinterpret_cast<float4*>(qs + i * LDK + 4 * c) = v;
    }
    const uint32_t j = tid % KC, ig = tid / KC;
    const bool scorer = ig < QT;  // false only for idle row groups (QT < GQ)
    const uint32_t x = tid % D, rg = tid / D;
    float4 kpre[NL], vpre[NL];
    auto fetch = [&](uint32_t c0) {
#pragma unroll
        for (uint32_t n = 0; n < NL; ++n) {
            const uint32_t e = tid + 256 * n;
            const uint32_t jj = e / (D / 4), c = e % (D / 4);
            kpre[n] = zero4;
            vpre[n] = zero4;
            if (c0 + jj < kend) {
                const size_t off = static_cast<size_t>(c0 + jj) * kvd + g * D + 4 * c;
                kpre[n] = *reinterpret_cast<const float4*>(kcache + off);
                vpre[n] = *reinterpret_cast<const float4*>(vcache + off);
            }
        }
    };
    fetch(0);
    float m_run[RQ], l_run[RQ], acc[RP];
#pragma unroll
    for (uint32_t m = 0; m < RQ; ++m) {
        m_run[m] = -INFINITY;
        l_run[m] = 0.0f;
    }
#pragma unroll
    for (uint32_t r = 0; r < RP; ++r) acc[r] = 0.0f;
    for (uint32_t c0 = 0; c0 < kend; c0 += KC) {
        __syncthreads();  // the previous chunk's ks / vs / ps / corr are consumed
#pragma unroll
        for (uint32_t n = 0; n < NL; ++n) {
            const uint32_t e = tid + 256 * n;
            const uint32_t jj = e / (D / 4), c = e % (D / 4);
            *reinterpret_cast<float4*>(ks + jj * LDK + 4 * c) = kpre[n];
            *reinterpret_cast<float4*>(vs + jj * D + 4 * c) = vpre[n];
        }
        __syncthreads();
        if (c0 + KC < kend) fetch(c0 + KC);
        float s[RQ];
#pragma unroll
        for (uint32_t m = 0; m < RQ; ++m) s[m] = 0.0f;
#pragma unroll 8
        for (uint32_t c = 0; c < D / 4; ++c) {
            const float4 kv = *reinterpret_cast<const float4*>(ks + j * LDK + 4 * c);
#pragma unroll
            for (uint32_t m = 0; m < RQ; ++m) {
                const float4 qv = *reinterpret_cast<const float4*>(qs + ((ig + GQ * m) % QT) * LDK + 4 * c);
                s[m] = fmaf(kv.x, qv.x, s[m]);
                s[m] = fmaf(kv.y, qv.y, s[m]);
                s[m] = fmaf(kv.z, qv.z, s[m]);
                s[m] = fmaf(kv.w, qv.w, s[m]);
            }
        }
        const uint32_t t = c0 + j;
#pragma unroll
        for (uint32_t m = 0; m < RQ; ++m) {
            const uint32_t i = ig + GQ * m;
            // key 0 is valid for every row, so m_new is finite from the first chunk on
            const float sv = t <= pos0 + r0 + i && t < kend ? s[m] * scale : -INFINITY;
            float cm = sv;
#pragma unroll
            for (uint32_t o = KC / 2; o > 0; o >>= 1) cm = fmaxf(cm, __shfl_xor(cm, o));
            const float m_new = fmaxf(m_run[m], cm);
            const float p = expf(sv - m_new);
            float cs = p;
#pragma unroll
            for (uint32_t o = KC / 2; o > 0; o >>= 1) cs += __shfl_xor(cs, o);
            const float cr = expf(m_run[m] - m_new);
            l_run[m] = l_run[m] * cr + cs;
            m_run[m] = m_new;
            if (scorer) {
                ps[j * QT + i] = p;
                if (j == 0) corr[i] = cr;
            }
        }
        __syncthreads();
#pragma unroll
        for (uint32_t r = 0; r < RP; ++r) acc[r] *= corr[rg * RP + r];
#pragma unroll 4
        for (uint32_t jj = 0; jj < KC; ++jj) {
            const float v = vs[jj * D + x];
#pragma unroll
            for (uint32_t r = 0; r < RP; ++r) acc[r] = fmaf(ps[jj * QT + rg * RP + r], v, acc[r]);
        }
    }
    if (j == 0 && scorer) {
#pragma unroll
        for (uint32_t m = 0; m < RQ; ++m) lsum[ig + GQ * m] = l_run[m];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t r = 0; r < RP; ++r) {
        const uint32_t i = rg * RP + r;
        if (i < nrow) out[static_cast<size_t>(r0 + i) * out_stride + h * D + x] = acc[r] / lsum[i];
    }
}

// ------------------------------------------------------------ argmax
// Ties resolve to the lower index; NaN never wins (strict '>').
__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

__device__ void block_argmax(float& bv, uint32_t& bi) {
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const uint32_t oi = __shfl_xor(bi, o);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    __shared__ float sv[16];
    __shared__ uint32_t si[16];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / 64; ++w) {
            if (better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        }
    }
}

__global__ __launch_bounds__(256) void argmax_partial(const float* __restrict__ x, uint32_t n, uint32_t per_block,
                                                      float* __restrict__ pv, uint32_t* __restrict__ pi) {
    const uint32_t b0 = blockIdx.x * per_block;
    const uint32_t b1 = min(n, b0 + per_block);
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t i = b0 + threadIdx.x; i < b1; i += blockDim.x) {
        const float v = x[i];
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    block_argmax(bv, bi);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(256) void argmax_final(const float* __restrict__ pv, const uint32_t* __restrict__ pi,
                                                    uint32_t parts, uint32_t* __restrict__ out) {
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t i = threadIdx.x; i < parts; i += blockDim.x) {
        if (better(pv[i], pi[i], bv, bi)) {
            bv = pv[i];
            bi = pi[i];
        }
    }
    block_argmax(bv, bi);
    if (threadIdx.x == 0) out[0] = bi;
}

// ------------------------------------------------------------ elementwise
// y = silu(g) * u with the reference's sign-branched sigmoid
// (cpu_llm.cpp:188-202), one thread per 16-group; optional XGroup form of y.
__global__ void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ y,
                              XGroup* __restrict__ yq, uint32_t n) {
    const uint32_t grp = blockIdx.x * blockDim.x + threadIdx.x;
    if (grp * 16 >= n) return;
    float v[16];
#pragma unroll
    for (uint32_t k = 0; k < 16; ++k) {
        const uint32_t i = 16 * grp + k;
        v[k] = 0.0f;
        if (i < n) {
            const float gate = g[i];
            const float sig = gate >= 0.0f ? 1.0f / (1.0f + expf(-gate)) : expf(gate) / (1.0f + expf(gate));
            v[k] = gate * sig * u[i];
            y[i] = v[k];
        }
    }
    if (yq) xgroup_encode(v, yq + grp);
}

__global__ void add_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ y, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a[i] + b[i];
}

}  // namespace

int launch_rmsnorm(const float* x, const float* gamma, float* y, XGroup* yq, size_t rows, size_t cols, float eps,
                   hipStream_t stream) {
    if (!x || !gamma || !y || rows == 0 || cols == 0) return kInvalidArgument;
    if (yq && (cols % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0)) return kInvalidArgument;
    if (cols % 4 == 0 && (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(y) % 16 != 0 ||
                          reinterpret_cast<uintptr_t>(gamma) % 16 != 0)) {
        return kInvalidArgument;
    }
    if (!(eps > 0.0f)) return kInvalidArgument;
    HIPLLM_LAUNCH(rmsnorm_kernel, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, stream, x, gamma, y, yq,
                       static_cast<uint32_t>(cols), eps);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

int launch_embed(uint32_t type, const void* table, size_t row_bytes, const int32_t* ids, size_t rows, size_t vocab,
                 size_t cols, float* out, hipStream_t stream) {
    if (!table || !ids || !out || rows == 0 || cols == 0 || vocab == 0) return kInvalidArgument;
    if (cols % block_elems(type) != 0) return kInvalidArgument;
    const dim3 grid(static_cast<uint32_t>((cols + 255) / 256), static_cast<uint32_t>(rows));
    HIPLLM_LAUNCH(embed_kernel, grid, dim3(256), 0, stream, type, static_cast<const uint8_t*>(table), row_bytes,
                       ids, static_cast<uint32_t>(vocab), static_cast<uint32_t>(cols), out);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

int launch_rope_kv(float* qkv, const float* cos_sin, size_t rot, size_t hq, size_t hkv, size_t d, size_t pos0,
                   size_t rows, size_t row_stride, float* kcache, float* vcache, hipStream_t stream,
                   const uint32_t* dpos) {
    if (!qkv || !cos_sin || !kcache || !vcache || rows == 0 || d == 0 || rot == 0 || rot > d || rot % 2) {
        return kInvalidArgument;
    }
    if (hq == 0 || hkv == 0 || hq % hkv != 0 || row_stride < (hq + 2 * hkv) * d) return kInvalidArgument;
    HIPLLM_LAUNCH(rope_kv_kernel, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, stream, qkv,
                       reinterpret_cast<const float2*>(cos_sin), static_cast<uint32_t>(rot / 2),
                       static_cast<uint32_t>(hq), static_cast<uint32_t>(hkv), static_cast<uint32_t>(d),
                       static_cast<uint32_t>(pos0), static_cast<uint32_t>(row_stride), kcache, vcache, dpos);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

namespace {
// Up to two chunks (one for heads of more than 128 dims) one block per head
// walks them all and writes the output (no merge launch): 28 heads of 128 at
// one chunk 5.5 us against 7.6 with the merge, at two 7.7 against 8.3, but
// each further chunk in turn costs about 2.5 us (11.4 against 8.8 at four),
// and heads of 256 at two chunks measured 10.9 against 9.5. Beyond, one
// split per chunk up to 16; the launchers run 2 to 4 splits of 64-, 128-
// or 256-dim heads as one block per head with the chunks side by side and
// the K (and V) loads issued first (28 heads of 128 at four chunks: 9.8 +
// 4.6 us as two launches, one launch about 5 us less).
uint32_t attn_splits(size_t max_len, size_t d) {
    const size_t chunks = (max_len + kAttnChunk - 1) / kAttnChunk;
    if (chunks <= (d > 128 ? 1u : 2u)) return 1;
    return static_cast<uint32_t>(chunks < kAttnMaxSplits ? chunks : kAttnMaxSplits);
}
}  // namespace

size_t attn_decode_scratch_floats(size_t hq, size_t d, size_t max_len) {
    return hq * attn_splits(max_len, d) * (d + 2);
}

// len > 0 keys, or (dpos != nullptr) len = *dpos + 1 read on the device with
// the split count of capacity keys (scratch sized by
// attn_decode_scratch_floats(hq, d, capacity); the caller guarantees
// *dpos < capacity).
int launch_attn_decode(const float* q, const float* kcache, const float* vcache, float* out, XGroup* outq,
                       float* scratch, size_t hq, size_t hkv, size_t d, size_t len, float scale, hipStream_t stream,
                       const uint32_t* dpos, size_t capacity) {
    if (!q || !kcache || !vcache || !out || !scratch || hq == 0 || hkv == 0 || hq % hkv) return kInvalidArgument;
    if (dpos ? capacity == 0 : len == 0) return kInvalidArgument;
    if (d == 0 || d > 256 || d % 16 != 0) return kInvalidArgument;
    if (outq && reinterpret_cast<uintptr_t>(outq) % 16 != 0) return kInvalidArgument;
    if (len > 0xffffffffull || capacity > 0xffffffffull || hq > 0xffffull) return kLengthError;
    const uint32_t splits = attn_splits(dpos ? capacity : len, d);
    // Read-only use of the caches (no RoPE table): the kernels write them only in the fused form.
    if (splits >= 2 && splits <= kAttnHeadChunks && (d == 64 || d == 128 || d == 256)) {
#define HIPLLM_ATTN_HEAD(D)                                                                                       \
    HIPLLM_LAUNCH((attn_decode_head<kAttnHeadChunks, D>), dim3(static_cast<uint32_t>(hq)), dim3(256 * kAttnHeadChunks), \
                  0, stream, q, const_cast<float*>(kcache), const_cast<float*>(vcache), static_cast<uint32_t>(hq),    \
                  static_cast<uint32_t>(hkv), static_cast<uint32_t>(len), dpos, scale, nullptr, 0u, out, outq, nullptr)
        if (d == 64) {
            HIPLLM_ATTN_HEAD(64);
        } else if (d == 128) {
            HIPLLM_ATTN_HEAD(128);
        } else {
            HIPLLM_ATTN_HEAD(256);
        }
#undef HIPLLM_ATTN_HEAD
        return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
    }
#define HIPLLM_ATTN_PARTIAL(DT)                                                                                   \
    HIPLLM_LAUNCH((attn_decode_partial<DT>), dim3(static_cast<uint32_t>(hq), splits), dim3(256), 0, stream, q,       \
                  const_cast<float*>(kcache), const_cast<float*>(vcache), scratch, static_cast<uint32_t>(hq),        \
                  static_cast<uint32_t>(hkv), static_cast<uint32_t>(d), static_cast<uint32_t>(len), dpos, scale,      \
                  splits, nullptr, 0u, out, outq, nullptr)
    if (d == 64) {
        HIPLLM_ATTN_PARTIAL(64);
    } else if (d == 128) {
        HIPLLM_ATTN_PARTIAL(128);
    } else {
        HIPLLM_ATTN_PARTIAL(0);
    }
#undef HIPLLM_ATTN_PARTIAL
    if (splits > 1) {
        HIPLLM_LAUNCH(attn_decode_merge, dim3(static_cast<uint32_t>(hq)), dim3(256), 0, stream, scratch, out,
                           outq, static_cast<uint32_t>(d), splits, nullptr);
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

// One decode token's RoPE, KV-cache write and attention: qkv is the token's
// raw [Q | K | V] row, the position is pos (len = pos + 1) or *dpos.
int launch_attn_decode_rope(const float* qkv, const float* cos_sin, size_t rot, float* kcache, float* vcache,
                            float* out, XGroup* outq, float* scratch, size_t hq, size_t hkv, size_t d, size_t pos,
                            float scale, hipStream_t stream, const uint32_t* dpos, size_t capacity,
                            const float* gate) {
    if (!qkv || !cos_sin || !kcache || !vcache || !out || !scratch || hq == 0 || hkv == 0 || hq % hkv) {
        return kInvalidArgument;
    }
    if (dpos && capacity == 0) return kInvalidArgument;
    if (d == 0 || d > 256 || d % 16 != 0 || rot == 0 || rot % 2 != 0 || rot > d) return kInvalidArgument;
    if (outq && reinterpret_cast<uintptr_t>(outq) % 16 != 0) return kInvalidArgument;
    if (pos >= 0xffffffffull || capacity > 0xffffffffull || hq > 0xffffull) return kLengthError;
    const uint32_t splits = attn_splits(dpos ? capacity : pos + 1, d);
    if (splits >= 2 && splits <= kAttnHeadChunks && (d == 64 || d == 128 || d == 256)) {
#define HIPLLM_ATTN_HEAD(D)                                                                                       \
    HIPLLM_LAUNCH((attn_decode_head<kAttnHeadChunks, D>), dim3(static_cast<uint32_t>(hq)), dim3(256 * kAttnHeadChunks), \
                  0, stream, qkv, kcache, vcache, static_cast<uint32_t>(hq), static_cast<uint32_t>(hkv),             \
                  static_cast<uint32_t>(pos + 1), dpos, scale, reinterpret_cast<const float2*>(cos_sin),              \
                  static_cast<uint32_t>(rot / 2), out, outq, gate)
        if (d == 64) {
            HIPLLM_ATTN_HEAD(64);
        } else if (d == 128) {
            HIPLLM_ATTN_HEAD(128);
        } else {
            HIPLLM_ATTN_HEAD(256);
        }
#undef HIPLLM_ATTN_HEAD
        return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
    }
#define HIPLLM_ATTN_PARTIAL(DT)                                                                                   \
    HIPLLM_LAUNCH((attn_decode_partial<DT>), dim3(static_cast<uint32_t>(hq), splits), dim3(256), 0, stream, qkv,     \
                  kcache, vcache, scratch, static_cast<uint32_t>(hq), static_cast<uint32_t>(hkv),                    \
                  static_cast<uint32_t>(d), static_cast<uint32_t>(pos + 1), dpos, scale, splits,                     \
                  reinterpret_cast<const float2*>(cos_sin), static_cast<uint32_t>(rot / 2), out, outq, gate)
    if (d == 64) {
        HIPLLM_ATTN_PARTIAL(64);
    } else if (d == 128) {
        HIPLLM_ATTN_PARTIAL(128);
    } else {
        HIPLLM_ATTN_PARTIAL(0);
    }
#undef HIPLLM_ATTN_PARTIAL
    if (splits > 1) {
        HIPLLM_LAUNCH(attn_decode_merge, dim3(static_cast<uint32_t>(hq)), dim3(256), 0, stream, scratch, out,
                           outq, static_cast<uint32_t>(d), splits, gate);
    }
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

bool attn_decode_qgate_fits(size_t max_len, size_t d) {
    const uint32_t splits = attn_splits(max_len, d);
    return splits >= 2 && splits <= kAttnHeadChunks && (d == 64 || d == 128 || d == 256);
}

int launch_attn_decode_qgate(const float* mixed, const float* kv, const float* q_gamma, const float* k_gamma,
                             float eps, const float* cos_sin, size_t rot, float* kcache, float* vcache, float* out,
                             XGroup* outq, size_t hq, size_t hkv, size_t d, size_t pos, float scale,
                             hipStream_t stream, const uint32_t* dpos, size_t capacity) {
    if (!mixed || !kv || !q_gamma || !k_gamma || !cos_sin || !kcache || !vcache || !out || hq == 0 || hkv == 0 ||
        hq % hkv || !(eps > 0.0f)) {
        return kInvalidArgument;
    }
    if (dpos && capacity == 0) return kInvalidArgument;
    if (rot == 0 || rot % 2 != 0 || rot > d) return kInvalidArgument;
    if (outq && reinterpret_cast<uintptr_t>(outq) % 16 != 0) return kInvalidArgument;
    if (pos >= 0xffffffffull || capacity > 0xffffffffull || hq > 0xffffull) return kLengthError;
    if (!attn_decode_qgate_fits(dpos ? capacity : pos + 1, d)) return kInvalidArgument;
    const AttnQGate qg{kv, q_gamma, k_gamma, eps};
#define HIPLLM_ATTN_QG(D)                                                                                          \
    HIPLLM_LAUNCH((attn_decode_head<kAttnHeadChunks, D, true>), dim3(static_cast<uint32_t>(hq)),                   \
                  dim3(256 * kAttnHeadChunks), 0, stream, mixed, kcache, vcache, static_cast<uint32_t>(hq),         \
                  static_cast<uint32_t>(hkv), static_cast<uint32_t>(pos + 1), dpos, scale,                        \
                  reinterpret_cast<const float2*>(cos_sin), static_cast<uint32_t>(rot / 2), out, outq, nullptr, qg)
    if (d == 64) {
        HIPLLM_ATTN_QG(64);
    } else if (d == 128) {
        HIPLLM_ATTN_QG(128);
    } else {
        HIPLLM_ATTN_QG(256);
    }
#undef HIPLLM_ATTN_QG
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

int launch_attn_prefill(const float* q, size_t q_stride, const float* kcache, const float* vcache, float* out,
                        size_t out_stride, size_t rows, size_t hq, size_t hkv, size_t d, size_t pos0, float scale,
                        hipStream_t stream) {
    if (!q || !kcache || !vcache || !out || rows == 0 || hq == 0 || hkv == 0 || hq % hkv) return kInvalidArgument;
    if (d == 0 || d > 256 || d % 4 != 0 || q_stride < hq * d || out_stride < hq * d) return kInvalidArgument;
    if (rows > 0x7fffffffull || hq > 0xffffull || pos0 + rows > 0xffffffffull) return kLengthError;
    if (d == 64 || d == 128 || d == 256) {
        // tiles of 16 rows once the grid holds two blocks per CU, else 8
        const bool wide = (rows + 15) / 16 * hq >= 512;
        const uint32_t qt = wide ? 16 : 8;
        const dim3 grid(static_cast<uint32_t>((rows + qt - 1) / qt), static_cast<uint32_t>(hq));
#define HIPLLM_ATTN_PF(D, QT)                                                                                     \
    HIPLLM_LAUNCH((attn_prefill_tiled_kernel<D, QT>), grid, dim3(256), 0, stream, q,                            \
                  static_cast<uint32_t>(q_stride), kcache, vcache, out, static_cast<uint32_t>(out_stride),       \
                  static_cast<uint32_t>(rows), static_cast<uint32_t>(hq), static_cast<uint32_t>(hkv),            \
                  static_cast<uint32_t>(pos0), scale)
        if (d == 64) {
            if (wide) HIPLLM_ATTN_PF(64, 16); else HIPLLM_ATTN_PF(64, 8);
        } else if (d == 128) {
            if (wide) HIPLLM_ATTN_PF(128, 16); else HIPLLM_ATTN_PF(128, 8);
        } else {
            if (wide) HIPLLM_ATTN_PF(256, 16); else HIPLLM_ATTN_PF(256, 8);
        }
#undef HIPLLM_ATTN_PF
        return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
    }
    HIPLLM_LAUNCH(attn_prefill_kernel, dim3(static_cast<uint32_t>(rows), static_cast<uint32_t>(hq)), dim3(256),
                       0, stream, q, static_cast<uint32_t>(q_stride), kcache, vcache, out,
                       static_cast<uint32_t>(out_stride), static_cast<uint32_t>(hq), static_cast<uint32_t>(hkv),
                       static_cast<uint32_t>(d), static_cast<uint32_t>(pos0), scale);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

constexpr uint32_t kArgmaxPerBlock = 2048;

size_t argmax_scratch_bytes(size_t n) {
    const size_t parts = (n + kArgmaxPerBlock - 1) / kArgmaxPerBlock;
    return parts * 8;
}

int launch_argmax(const float* x, size_t n, uint32_t* out, void* scratch, hipStream_t stream) {
    if (!x || !out || !scratch || n == 0 || n > 0xffffffffull) return kInvalidArgument;
    const uint32_t parts = static_cast<uint32_t>((n + kArgmaxPerBlock - 1) / kArgmaxPerBlock);
    float* pv = static_cast<float*>(scratch);
    uint32_t* pi = reinterpret_cast<uint32_t*>(pv + parts);
    HIPLLM_LAUNCH(argmax_partial, dim3(parts), dim3(256), 0, stream, x, static_cast<uint32_t>(n),
                       kArgmaxPerBlock, pv, pi);
    HIPLLM_LAUNCH(argmax_final, dim3(1), dim3(256), 0, stream, pv, pi, parts, out);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

int launch_swiglu(const float* g, const float* u, float* y, XGroup* yq, size_t n, hipStream_t stream) {
    if (!g || !u || !y || n == 0 || (yq && (n % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0))) {
        return kInvalidArgument;
    }
    const uint32_t groups = static_cast<uint32_t>((n + 15) / 16);
    HIPLLM_LAUNCH(swiglu_kernel, dim3((groups + 255) / 256), dim3(256), 0, stream, g, u, y, yq,
                       static_cast<uint32_t>(n));
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

int launch_add(const float* a, const float* b, float* y, size_t n, hipStream_t stream) {
    if (!a || !b || !y || n == 0) return kInvalidArgument;
    HIPLLM_LAUNCH(add_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, stream, a, b, y, n);
    return hipGetLastError() == hipSuccess ? kOk : kRuntimeError;
}

}  // namespace hipllm
