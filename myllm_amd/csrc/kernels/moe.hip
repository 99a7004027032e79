// qwen35moe operators: router top-k, MoE combine, Gated DeltaNet (gates,
// causal conv + SiLU + history, L2 head norm, the recurrent state scan, gated
// RMSNorm) and the gated full-attention pieces (Q/gate split with per-head
// RMSNorm, sigmoid output gate).
//
// Reference semantics (MoeLLM, moe_llm.mm:2238-2843, and its kernels):
//   router        softmax metal_llm.metal:826-890, top-k insertion 1424-1459
//                 (strict '>': lower expert id wins ties), renorm 1461-1474
//   combine       weighted reduce 1525-1542, shared gate 1186-1197 +
//                 row scale 1265-1276, residuals (moe_llm.mm:2836-2885)
//   DeltaNet      softplus 1213-1224, exp 1226-1233, conv 1320-1341, history
//                 1345-1365, SiLU 1199-1211, L2 norm 1280-1316, recurrence
//                 1370-1420, per-head RMSNorm 785-823 times SiLU(z)
//   attention     Q/gate split 1167-1184, per-head RMSNorm 785-823, sigmoid
//                 gate + multiply (moe_llm.mm:2420-2428)
//
// Design for CDNA4: the DeltaNet scan keeps each value head's 128 x 128 FP32
// state in registers for the whole prompt (one block per head and 64-column
// tile, 256 threads, 32 state values per thread) so the state is read and
// written once per call however many tokens it scans; norms run one 64-lane
// wave per head vector; everything else is one pass over its rows.
#include <algorithm>

#include "common.h"
#include "launch.h"
#include "norm.h"
#include "router.h"

namespace hipllm {
namespace {

__device__ __forceinline__ float softplus_ref(float v) {
    return v > 20.0f ? v : (v < -20.0f ? expf(v) : logf(1.0f + expf(v)));
}


// ------------------------------------------------------------ router
template <uint32_t PL>
__global__ __launch_bounds__(64) void router_topk_kernel(const float* __restrict__ logits, uint32_t ld,
                                                         uint32_t experts, uint32_t k, int32_t* __restrict__ ids,
                                                         float* __restrict__ weights) {
    const size_t t = blockIdx.x;
    topk_row<PL>(logits + t * ld, experts, k, ids + t * k, weights + t * k, threadIdx.x);
}

// ------------------------------------------------------------ router over a prompt
// y[m, n] = x[m, :k] . w[n, :k] in FP32 (the router logits of a prompt; the
// batched GEMV reads every weight row once per token). Block tile 32 rows x
// 32 weight rows, 256 threads with 2 x 2 outputs each; k staged through LDS
// 128 at a time (k-major, so a thread reads its two rows / columns as one
// float2), the next step's values loaded while this step multiplies. Block z
// covers k range [z kc, (z + 1) kc) (grid z = the K split; with a split it
// writes partial sums to part[z], which matmul_reduce_kernel adds in z
// order). Each output sums its k range in increasing order, one FMA per
// step: deterministic. A block's time is its FMA chains (about 50 us for
// k = 2048 unsplit), so the split fills the GPU.
constexpr uint32_t kMmTile = 32, kMmK = 128;

__global__ __launch_bounds__(256) void matmul_f32_kernel(const float* __restrict__ x, uint32_t ldx,
                                                         const float* __restrict__ w, uint32_t ldw,
                                                         float* __restrict__ y, uint32_t ldy, uint32_t m,
                                                         uint32_t n, uint32_t k, uint32_t kc,
                                                         float* __restrict__ part) {
    __shared__ __align__(16) float xs[kMmK][kMmTile + 2];
    __shared__ __align__(16) float ws[kMmK][kMmTile + 2];
    constexpr uint32_t kPer = kMmK / 8;  // k values a thread moves per row per step
    const uint32_t tid = threadIdx.x;
    const uint32_t m0 = blockIdx.y * kMmTile, n0 = blockIdx.x * kMmTile;
    const uint32_t tm = (tid / 16) * 2, tn = (tid % 16) * 2;  // this thread's 2 x 2 outputs
    // Loader: thread t moves k columns kPer (t % 8) .. + kPer of row t / 8.
    const uint32_t lr = tid / 8, lc = kPer * (tid % 8);
    const bool xrow = m0 + lr < m, wrow = n0 + lr < n;
    const float* xp = x + static_cast<size_t>(min(m0 + lr, m - 1)) * ldx;
    const float* wp = w + static_cast<size_t>(min(n0 + lr, n - 1)) * ldw;
    const bool vec = (ldx % 4 == 0) && (ldw % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                     (reinterpret_cast<uintptr_t>(w) % 16 == 0);
    auto load = [&](uint32_t k0, float (&xv)[kPer], float (&wv)[kPer]) {
        const uint32_t kb = k0 + lc;
        if (vec && kb + kPer <= k) {
#pragma unroll
            for (uint32_t i = 0; i < kPer / 4; ++i) {
                const float4 a = xrow ? *reinterpret_cast<const float4*>(xp + kb + 4 * i) : make_float4(0, 0, 0, 0);
                const float4 b = wrow ? *reinterpret_cast<const float4*>(wp + kb + 4 * i) : make_float4(0, 0, 0, 0);
                xv[4 * i] = a.x, xv[4 * i + 1] = a.y, xv[4 * i + 2] = a.z, xv[4 * i + 3] = a.w;
                wv[4 * i] = b.x, wv[4 * i + 1] = b.y, wv[4 * i + 2] = b.z, wv[4 * i + 3] = b.w;
            }
        } else {
#pragma unroll
            for (uint32_t i = 0; i < kPer; ++i) {
                xv[i] = (xrow && kb + i < k) ? xp[kb + i] : 0.0f;
                wv[i] = (wrow && kb + i < k) ? wp[kb + i] : 0.0f;
            }
        }
    };
    float acc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
    float xv[kPer], wv[kPer];
    const uint32_t kbeg = blockIdx.z * kc, kend = min(k, kbeg + kc);
    load(kbeg, xv, wv);
    for (uint32_t k0 = kbeg; k0 < kend; k0 += kMmK) {
        __syncthreads();  // the previous step's reads are done
#pragma unroll
        for (uint32_t i = 0; i < kPer; ++i) {
            xs[lc + i][lr] = xv[i];
            ws[lc + i][lr] = wv[i];
        }
        __syncthreads();
        if (k0 + kMmK < kend) load(k0 + kMmK, xv, wv);
        const uint32_t steps = min(kMmK, kend - k0);
        for (uint32_t kk = 0; kk < steps; ++kk) {
            const float2 a = *reinterpret_cast<const float2*>(&xs[kk][tm]);
            const float2 b = *reinterpret_cast<const float2*>(&ws[kk][tn]);
            acc[0][0] = fmaf(a.x, b.x, acc[0][0]);
            acc[0][1] = fmaf(a.x, b.y, acc[0][1]);
            acc[1][0] = fmaf(a.y, b.x, acc[1][0]);
            acc[1][1] = fmaf(a.y, b.y, acc[1][1]);
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i) {
#pragma unroll
        for (uint32_t j = 0; j < 2; ++j) {
            if (m0 + tm + i < m && n0 + tn + j < n) {
                if (part) {
                    part[(static_cast<size_t>(blockIdx.z) * m + m0 + tm + i) * n + n0 + tn + j] = acc[i][j];
                } else {
                    y[static_cast<size_t>(m0 + tm + i) * ldy + n0 + tn + j] = acc[i][j];
                }
            }
        }
    }
}

// y[r, c] = sum over z in order of part[z, r, c].
__global__ void matmul_reduce_kernel(const float* __restrict__ part, float* __restrict__ y, uint32_t ldy, uint32_t m,
                                     uint32_t n, uint32_t splits) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t total = static_cast<size_t>(m) * n;
    if (i >= total) return;
    float acc = part[i];
    for (uint32_t z = 1; z < splits; ++z) acc += part[z * total + i];
    y[(i / n) * ldy + i % n] = acc;
}

// ------------------------------------------------------------ route groups
// Counting sort of n routed vectors by expert in one block, then the expert
// groups of at most vmax vectors: per-expert counts with LDS atomics, one
// thread turns them into offsets (vectors and groups), every vector takes
// the next slot of its expert (LDS atomic), and thread e writes expert e's
// groups. The order of the vectors inside one expert follows the atomics;
// it changes nothing downstream, where every vector's row is computed on its
// own (its X row against the expert's weights, written to its own y row).
// O(n + experts); a scan of all ids per expert measured 284 us at 4096 x 256.
constexpr uint32_t kRouteGroupsMax = 16384;

__global__ __launch_bounds__(1024) void route_groups_kernel(const int32_t* __restrict__ ids, uint32_t n,
                                                            uint32_t experts, uint32_t vmax,
                                                            int32_t* __restrict__ order,
                                                            int32_t* __restrict__ groups,
                                                            uint32_t* __restrict__ ngroups) {
    // One expert per thread (experts <= kMaxExperts == blockDim.x): the
    // vector and group offsets are exclusive prefix sums over experts, a
    // shuffle scan per wave and one over the wave totals.
    __shared__ uint32_t cnt[kMaxExperts];
    __shared__ uint32_t cur[kMaxExperts];
    __shared__ uint32_t wtot[2][kMaxExperts / 64];
    const uint32_t e = threadIdx.x, lane = e & 63, wave = e >> 6;
    if (e < experts) cnt[e] = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        atomicAdd(&cnt[min(static_cast<uint32_t>(ids[i]), experts - 1)], 1u);
    }
    __syncthreads();
    const uint32_t c = e < experts ? cnt[e] : 0;
    const uint32_t gc = (c + vmax - 1) / vmax;
    uint32_t run = c, grun = gc;  // inclusive within the wave
#pragma unroll
    for (uint32_t o = 1; o < 64; o <<= 1) {
        const uint32_t r = __shfl_up(run, o, 64), gr = __shfl_up(grun, o, 64);
        if (lane >= o) {
            run += r;
            grun += gr;
        }
    }
    if (lane == 63) {
        wtot[0][wave] = run;
        wtot[1][wave] = grun;
    }
    __syncthreads();
    uint32_t base = 0, gbase = 0;
    for (uint32_t w = 0; w < wave; ++w) {
        base += wtot[0][w];
        gbase += wtot[1][w];
    }
    const uint32_t start = base + run - c, gstart = gbase + grun - gc;
    if (e < experts) cur[e] = start;
    if (e == experts - 1) *ngroups = gstart + gc;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const uint32_t slot = atomicAdd(&cur[min(static_cast<uint32_t>(ids[i]), experts - 1)], 1u);
        order[slot] = static_cast<int32_t>(i);
    }
    for (uint32_t q = 0; q < gc; ++q) {
        groups[2 * (gstart + q)] = static_cast<int32_t>(start + q * vmax);
        groups[2 * (gstart + q) + 1] = static_cast<int32_t>(e | (min(vmax, c - q * vmax) << 16));
    }
}

// ------------------------------------------------------------ MoE combine
// out[t] = residual[t] + (sum_r w[t, r] * down[t k + r] + sigmoid(sg[t]) * shared[t])
__device__ __forceinline__ float moe_combine_value(const float* __restrict__ residual, const float* __restrict__ down,
                                                   const float* __restrict__ w, const float* __restrict__ shared,
                                                   const float* __restrict__ sgate, uint32_t ld_sgate, uint32_t t,
                                                   uint32_t c, uint32_t h, uint32_t k) {
    const size_t i = static_cast<size_t>(t) * h + c;
    float acc = 0.0f;
    for (uint32_t r = 0; r < k; ++r) acc += w[t * k + r] * down[(static_cast<size_t>(t) * k + r) * h + c];
    float moe = acc;
    if (shared) moe += shared[i] * sigmoid_ref(sgate[static_cast<size_t>(t) * ld_sgate]);
    return residual[i] + moe;
}

__global__ void moe_combine_kernel(const float* __restrict__ residual, const float* __restrict__ down,
                                   const float* __restrict__ w, const float* __restrict__ shared,
                                   const float* __restrict__ sgate, uint32_t ld_sgate, float* __restrict__ out,
                                   uint32_t tokens, uint32_t h, uint32_t k) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<size_t>(tokens) * h) return;
    const uint32_t t = static_cast<uint32_t>(i / h), c = static_cast<uint32_t>(i % h);
    out[i] = moe_combine_value(residual, down, w, shared, sgate, ld_sgate, t, c, h, k);
}

constexpr uint32_t kCombineMaxK = 8;  // routes held in registers by the vector form

// The combine of one token per block, then the RMSNorm of the finished row
// (the next layer's input norm, or the output norm) by the same block, with
// the standalone norm kernel's arithmetic and block size.
__global__ __launch_bounds__(256) void moe_combine_norm_kernel(
    const float* __restrict__ residual, const float* __restrict__ down, const float* __restrict__ w,
    const float* __restrict__ shared, const float* __restrict__ sgate, uint32_t ld_sgate, float* out,
    const float* __restrict__ gamma, float* __restrict__ norm, XGroup* __restrict__ normq, uint32_t h, uint32_t k,
    float eps) {
    const uint32_t t = blockIdx.x;
    float* row = out + static_cast<size_t>(t) * h;
    if (h % 4 == 0 && k <= kCombineMaxK) {
        // float4 columns with every route's load issued before the sums (the
        // per-column form waits on k loads in turn); the same operations in
        // the same order per element as moe_combine_value.
        const uint32_t h4 = h / 4;
        float wt[kCombineMaxK];
#pragma unroll
        for (uint32_t r = 0; r < kCombineMaxK; ++r) wt[r] = r < k ? w[t * k + r] : 0.0f;
        const float sg = shared ? sigmoid_ref(sgate[static_cast<size_t>(t) * ld_sgate]) : 0.0f;
        const float4* d4 = reinterpret_cast<const float4*>(down) + static_cast<size_t>(t) * k * h4;
        const float4* r4 = reinterpret_cast<const float4*>(residual) + static_cast<size_t>(t) * h4;
        const float4* s4 = reinterpret_cast<const float4*>(shared) + static_cast<size_t>(t) * h4;
        for (uint32_t c = threadIdx.x; c < h4; c += blockDim.x) {
            float4 dv[kCombineMaxK];
#pragma unroll
            for (uint32_t r = 0; r < kCombineMaxK; ++r) {
                if (r < k) dv[r] = d4[static_cast<size_t>(r) * h4 + c];
            }
            const float4 res = r4[c];
            const float4 sh = shared ? s4[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t r = 0; r < kCombineMaxK; ++r) {
                if (r < k) {
                    a[0] += wt[r] * dv[r].x;
                    a[1] += wt[r] * dv[r].y;
                    a[2] += wt[r] * dv[r].z;
                    a[3] += wt[r] * dv[r].w;
                }
            }
            if (shared) {
                a[0] += sh.x * sg;
                a[1] += sh.y * sg;
                a[2] += sh.z * sg;
                a[3] += sh.w * sg;
            }
            reinterpret_cast<float4*>(row)[c] = make_float4(res.x + a[0], res.y + a[1], res.z + a[2], res.w + a[3]);
        }
    } else {
        for (uint32_t c = threadIdx.x; c < h; c += blockDim.x) {
            row[c] = moe_combine_value(residual, down, w, shared, sgate, ld_sgate, t, c, h, k);
        }
    }
    __syncthreads();
    rmsnorm_row(row, gamma, norm + static_cast<size_t>(t) * h, normq ? normq + static_cast<size_t>(t) * (h / 16) : nullptr,
                h, eps);
}

// ------------------------------------------------------------ DeltaNet
// decay = exp(softplus(alpha + dt_bias) * a), beta = sigmoid(beta_raw).
__global__ void gdn_gates_kernel(const float* __restrict__ alpha, const float* __restrict__ beta_raw, uint32_t ld,
                                 const float* __restrict__ dt_bias, const float* __restrict__ a,
                                 float* __restrict__ decay, float* __restrict__ beta, uint32_t tokens,
                                 uint32_t heads) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= tokens * heads) return;
    const uint32_t t = i / heads, h = i % heads;
    const float sp = softplus_ref(alpha[t * ld + h] + dt_bias[h]);
    decay[i] = expf(sp * a[h]);
    beta[i] = sigmoid_ref(beta_raw[t * ld + h]);
}

// Causal depthwise conv + SiLU over [history (k - 1 rows); x rows], then the
// history keeps the last k - 1 rows. One thread owns one channel for all
// tokens, so the history is read before it is overwritten.
constexpr uint32_t kMaxConv = 9;

// Block (64 channels, 16-token chunk); thread (channel lane, sub) computes
// tokens chunk * 16 + sub + 4 j (j < 4), each from its own window, so every
// load is independent (one thread per channel walking the tokens in turn
// measured 42 us for 64 tokens x 8192 channels). Only the chunk-0 blocks read
// the history (chunks are at least ksize - 1 tokens long, so later chunks
// never need it), and they alone write the new history of their channels,
// after a barrier: no block overwrites a row another still needs. Each output
// is the same sum in the same order as a sliding window.
constexpr uint32_t kConvChunk = 16;

__global__ __launch_bounds__(256) void conv1d_silu_kernel(const float* __restrict__ x, uint32_t ldx,
                                                          float* __restrict__ history, const float* __restrict__ w,
                                                          float* __restrict__ out, uint32_t ldo, uint32_t tokens,
                                                          uint32_t channels, uint32_t ksize) {
    const uint32_t c = blockIdx.x * 64 + (threadIdx.x & 63);
    const uint32_t sub = threadIdx.x >> 6;
    const uint32_t hr = ksize - 1;
    const bool live = c < channels;
    if (live) {
        float taps[kMaxConv];
        for (uint32_t i = 0; i < ksize; ++i) taps[i] = w[static_cast<size_t>(c) * ksize + i];
#pragma unroll
        for (uint32_t jj = 0; jj < kConvChunk / 4; ++jj) {
            const uint32_t t = blockIdx.y * kConvChunk + sub + 4 * jj;
            if (t >= tokens) break;
            float acc = 0.0f;
            for (uint32_t i = 0; i < ksize; ++i) {
                // input at time t - hr + i: a prompt row, or history row (t + i) when negative
                const float v = t + i >= hr ? x[static_cast<size_t>(t + i - hr) * ldx + c]
                                            : history[static_cast<size_t>(t + i) * channels + c];
                acc += v * taps[i];
            }
            out[static_cast<size_t>(t) * ldo + c] = acc * sigmoid_ref(acc);
        }
    }
    if (blockIdx.y != 0) return;
    __syncthreads();  // every read of the old history in this block is done
    if (!live || sub != 0) return;
    // New history row i = input at time tokens - hr + i.
    float nh[kMaxConv];
    for (uint32_t i = 0; i < hr; ++i) {
        nh[i] = tokens + i >= hr ? x[static_cast<size_t>(tokens + i - hr) * ldx + c]
                                 : history[static_cast<size_t>(tokens + i) * channels + c];
    }
    for (uint32_t i = 0; i < hr; ++i) history[static_cast<size_t>(i) * channels + c] = nh[i];
}

// x <- x * rsqrt(sum(x^2) + eps) for `heads` vectors of d values per row.
// One wave per (row, head).
__global__ __launch_bounds__(64) void l2norm_heads_kernel(float* __restrict__ x, uint32_t ld, uint32_t d,
                                                         float eps) {
    const uint32_t t = blockIdx.x, h = blockIdx.y;
    float* v = x + static_cast<size_t>(t) * ld + static_cast<size_t>(h) * d;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < d; i += 64) ss += v[i] * v[i];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss + eps);
    for (uint32_t i = threadIdx.x; i < d; i += 64) v[i] = v[i] * inv;
}

// Gated DeltaNet scan. Column j of the state S_h[Dk][Dv] (row = key dim)
// evolves on its own: per token, with key head h % key_heads,
// S[:, j] *= decay; pred_j = S[:, j] . k; delta_j = beta (v_j - pred_j);
// S[:, j] += k delta_j; o_j = S[:, j] . q / sqrt(Dk). So a block is one wave
// of four columns of one value head: lane 16 c + r holds rows
// [r NR, r NR + NR) of column c (NR = D / 16), both column sums are 16-lane
// DPP reductions, and no token needs a block barrier. Each token's inputs
// are loaded eight tokens ahead of its recurrence. Blocks are
// renumbered so that every XCD (which receives every eighth block) runs the
// columns of whole key heads, whose k and q rows its L2 then holds.
template <uint32_t D, bool VEC>
__global__ __launch_bounds__(64) void gdn_scan_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                      uint32_t ldqk, const float* __restrict__ v, uint32_t ldv,
                                                      const float* __restrict__ decay,
                                                      const float* __restrict__ beta, float* __restrict__ state,
                                                      float* __restrict__ out, uint32_t ldo, uint32_t tokens,
                                                      uint32_t value_heads, uint32_t key_heads) {
    constexpr uint32_t NR = D / 16, WPH = D / 4;  // rows per lane, blocks per value head
    const uint32_t nb = gridDim.x;
    const uint32_t b = nb % 8 == 0 ? (blockIdx.x % 8) * (nb / 8) + blockIdx.x / 8 : blockIdx.x;
    const uint32_t ratio = value_heads / key_heads;
    const uint32_t lh = b / WPH;  // value heads of one key head are adjacent in this order
    const uint32_t kh = lh / ratio, h = (lh % ratio) * key_heads + kh;
    const uint32_t r = threadIdx.x & 15;
    const uint32_t col = (b % WPH) * 4 + (threadIdx.x >> 4);
    float* S = state + static_cast<size_t>(h) * D * D;
    float s[NR];
#pragma unroll
    for (uint32_t i = 0; i < NR; ++i) s[i] = S[static_cast<size_t>(r * NR + i) * D + col];
    const float qscale = 1.0f / sqrtf(static_cast<float>(D));
    // Ring of the next PF tokens' inputs in registers: a step takes about a
    // tenth of a load's latency, so the loads run PF tokens ahead.
    constexpr uint32_t PF = 8;
    float kb[PF][NR], qb[PF][NR], vb[PF], gb[PF], bb[PF];
    auto load = [&](uint32_t t, float (&kk)[NR], float (&qq)[NR], float& vv, float& gg, float& bt) {
        const size_t off = static_cast<size_t>(t) * ldqk + kh * D + r * NR;
        if constexpr (VEC) {
#pragma unroll
            for (uint32_t i = 0; i < NR; i += 4) {
                const float4 a = *reinterpret_cast<const float4*>(k + off + i);
                const float4 c = *reinterpret_cast<const float4*>(q + off + i);
                kk[i] = a.x, kk[i + 1] = a.y, kk[i + 2] = a.z, kk[i + 3] = a.w;
                qq[i] = c.x, qq[i + 1] = c.y, qq[i + 2] = c.z, qq[i + 3] = c.w;
            }
        } else {
#pragma unroll
            for (uint32_t i = 0; i < NR; ++i) kk[i] = k[off + i], qq[i] = q[off + i];
        }
        vv = v[static_cast<size_t>(t) * ldv + h * D + col];
        gg = decay[static_cast<size_t>(t) * value_heads + h];
        bt = beta[static_cast<size_t>(t) * value_heads + h];
    };
#pragma unroll
    for (uint32_t p = 0; p < PF; ++p) {
        if (p < tokens) load(p, kb[p], qb[p], vb[p], gb[p], bb[p]);
    }
    for (uint32_t t0 = 0; t0 < tokens; t0 += PF) {
#pragma unroll
        for (uint32_t p = 0; p < PF; ++p) {
            const uint32_t t = t0 + p;
            if (t < tokens) {
                float pp = 0.0f;
#pragma unroll
                for (uint32_t i = 0; i < NR; ++i) {
                    s[i] *= gb[p];
                    pp += s[i] * kb[p][i];
                }
                const float pred = row16_sum(pp);
                const float delta = bb[p] * (vb[p] - pred);
                float op = 0.0f;
#pragma unroll
                for (uint32_t i = 0; i < NR; ++i) {
                    s[i] += kb[p][i] * delta;
                    op += s[i] * qb[p][i];
                }
                const float o = row16_sum(op);
                if (r == 0) out[static_cast<size_t>(t) * ldo + h * D + col] = o * qscale;
                if (t + PF < tokens) load(t + PF, kb[p], qb[p], vb[p], gb[p], bb[p]);
            }
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < NR; ++i) S[static_cast<size_t>(r * NR + i) * D + col] = s[i];
}

// Chunked Gated DeltaNet scan for prompts: the recurrence of gdn_scan_kernel
// over chunks of C = 64 tokens, the chunk-parallel (WY) form of the delta
// rule. Within a chunk starting from state S0, with G_t the cumulative log
// decay (G_t = sum of log decay_i, i <= t), the per-token deltas
// delta_t = beta_t (v_t - k_t . S_{t-1}-decayed) satisfy
//   (I + A) Delta = R,  A[t][i] = beta_t exp(G_t - G_i) (k_t . k_i) (i < t),
//                       R[t]    = beta_t (v_t - exp(G_t) S0^T k_t),
// the outputs are o_t = (exp(G_t) S0^T q_t + sum_{i<=t} exp(G_t - G_i)
// (q_t . k_i) delta_i) / sqrt(D), and the chunk ends in
//   S = exp(G_last) S0 + sum_t exp(G_last - G_t) k_t delta_t^T.
// Every exponent is <= 0. gdn_chunk_prep_kernel builds, for each (value
// head, chunk) at once, T = (I + A)^-1 and P[t][i] = exp(G_t - G_i)
// (q_t . k_i) (i <= t); gdn_chunk_scan_kernel then walks the chunks in order
// for 16 state columns per block (the columns evolve independently), so the
// serial part is one chunk step per 64 tokens. Rows past the prompt's end are
// zero keys with beta 0 and decay 1, which leave everything unchanged.
constexpr uint32_t kChunk = 64;
constexpr uint32_t kChunkCols = 16;

// G_t (cumulative log decay) and beta_t of one chunk into LDS: the first
// wave, lane t for token t, an inclusive prefix sum over the wave in a fixed
// order (both chunk kernels compute the same bits).
__device__ __forceinline__ void chunk_gates(const float* __restrict__ decay, const float* __restrict__ beta,
                                            uint32_t value_heads, uint32_t h, uint32_t t0, uint32_t len,
                                            float* G, float* B) {
    if (threadIdx.x < kChunk) {
        const uint32_t t = threadIdx.x;
        float g = 0.0f, b = 0.0f;
        if (t < len) {
            const float dc = decay[static_cast<size_t>(t0 + t) * value_heads + h];
            g = dc > 0.0f ? logf(dc) : -87.0f;  // decay 0 (underflow) as e^-87
            b = beta[static_cast<size_t>(t0 + t) * value_heads + h];
        }
#pragma unroll
        for (uint32_t off = 1; off < kChunk; off *= 2) {
            const float up = __shfl_up(g, off, 64);
            if (t >= off) g += up;
        }
        G[t] = g;
        B[t] = b;
    }
}

// Rows [t0, t0 + 64) of a [tokens, ld] matrix, columns col0 + [0, D), into
// LDS (rows past len are zero). All of a thread's loads issue before its LDS
// stores: VEC (16-byte aligned rows) as float4, otherwise as scalars.
template <uint32_t D, bool VEC>
__device__ __forceinline__ void chunk_rows(const float* __restrict__ src, uint32_t ld, uint32_t col0, uint32_t t0,
                                           uint32_t len, float (*dst)[D + 1]) {
    constexpr uint32_t N4 = kChunk * D / 4 / 256;  // float4 per thread
    float4 r[N4];
#pragma unroll
    for (uint32_t n = 0; n < N4; ++n) {
        const uint32_t i = threadIdx.x + 256 * n, t = i / (D / 4), d = 4 * (i % (D / 4));
        const float* p = src + static_cast<size_t>(t0 + t) * ld + col0 + d;
        if (t >= len) {
            r[n] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        } else if constexpr (VEC) {
            r[n] = *reinterpret_cast<const float4*>(p);
        } else {
            r[n] = make_float4(p[0], p[1], p[2], p[3]);
        }
    }
#pragma unroll
    for (uint32_t n = 0; n < N4; ++n) {
        const uint32_t i = threadIdx.x + 256 * n, t = i / (D / 4), d = 4 * (i % (D / 4));
        dst[t][d] = r[n].x, dst[t][d + 1] = r[n].y, dst[t][d + 2] = r[n].z, dst[t][d + 3] = r[n].w;
    }
}

template <uint32_t D, bool VEC>
__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                             uint32_t ldqk, const float* __restrict__ decay,
                                                             const float* __restrict__ beta,
                                                             float* __restrict__ tp, uint32_t tokens,
                                                             uint32_t value_heads, uint32_t key_heads) {
    const uint32_t h = blockIdx.x, c = blockIdx.y, kh = h % key_heads;
    const uint32_t t0 = c * kChunk, len = min(kChunk, tokens - t0);
    __shared__ float Ks[kChunk][D + 1], Qs[kChunk][D + 1];
    __shared__ float As[kChunk][kChunk + 4];
    __shared__ float G[kChunk], B[kChunk];
    chunk_rows<D, VEC>(k, ldqk, kh * D, t0, len, Ks);
    chunk_rows<D, VEC>(q, ldqk, kh * D, t0, len, Qs);
    chunk_gates(decay, beta, value_heads, h, t0, len, G, B);
    __syncthreads();
    // 4 x 4 (t, i) tile per thread of K K^T and Q K^T.
    const uint32_t tt = threadIdx.x / 16, ii = threadIdx.x % 16;
    float kk[4][4] = {}, qk[4][4] = {};
    for (uint32_t d = 0; d < D; ++d) {
        float kt[4], qt[4], ki[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            kt[a] = Ks[4 * tt + a][d];
            qt[a] = Qs[4 * tt + a][d];
            ki[a] = Ks[4 * ii + a][d];
        }
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                kk[a][b] = fmaf(kt[a], ki[b], kk[a][b]);
                qk[a][b] = fmaf(qt[a], ki[b], qk[a][b]);
            }
    }
    float* T = tp + (static_cast<size_t>(c) * value_heads + h) * 2 * kChunk * kChunk;
    float* P = T + kChunk * kChunk;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t t = 4 * tt + a, i = 4 * ii + b;
            const float dec = i <= t ? expf(G[t] - G[i]) : 0.0f;
            As[t][i] = i < t ? B[t] * dec * kk[a][b] : 0.0f;
            P[t * kChunk + i] = dec * qk[a][b];
        }
    __syncthreads();
    // T = (I + A)^-1 by forward substitution, one column per lane of the
    // first wave (T is unit lower triangular): T[t][j] = [t == j] -
    // sum_{i < t} A[t][i] T[i][j], every A[t][i] an LDS broadcast; four
    // partial sums (i mod 4) shorten the dependent chain.
    if (threadIdx.x < kChunk) {
        const uint32_t j = threadIdx.x;
        float col[kChunk];
#pragma unroll
        for (uint32_t t = 0; t < kChunk; ++t) {
            float a4[4] = {t == j ? 1.0f : 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t i = 0; i < t; ++i) a4[i % 4] = fmaf(-As[t][i], col[i], a4[i % 4]);
            const float acc = (a4[0] + a4[1]) + (a4[2] + a4[3]);
            col[t] = acc;
            T[t * kChunk + j] = acc;
        }
    }
}

// Block (value head h, column group cg) owns state columns
// [16 cg, 16 cg + 16) of head h and walks the chunks in order.
template <uint32_t D, bool VEC>
__global__ __launch_bounds__(256) void gdn_chunk_scan_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                             uint32_t ldqk, const float* __restrict__ v, uint32_t ldv,
                                                             const float* __restrict__ decay,
                                                             const float* __restrict__ beta,
                                                             const float* __restrict__ tp, float* __restrict__ state,
                                                             float* __restrict__ out, uint32_t ldo, uint32_t tokens,
                                                             uint32_t value_heads, uint32_t key_heads) {
    constexpr uint32_t CG = D / kChunkCols;
    const uint32_t h = blockIdx.x / CG, col0 = (blockIdx.x % CG) * kChunkCols, kh = h % key_heads;
    const uint32_t tid = threadIdx.x;
    __shared__ float Ks[kChunk][D + 1], Qs[kChunk][D + 1];
    __shared__ float Ts[kChunk][kChunk + 1], Ps[kChunk][kChunk + 1];
    __shared__ float Ss[D][kChunkCols];
    __shared__ float Rs[kChunk][kChunkCols + 1], Ds[kChunk][kChunkCols + 1];
    __shared__ float G[kChunk], B[kChunk], E[kChunk];
    float* S = state + static_cast<size_t>(h) * D * D;
    for (uint32_t i = tid; i < D * kChunkCols; i += 256) {
        Ss[i / kChunkCols][i % kChunkCols] = S[static_cast<size_t>(i / kChunkCols) * D + col0 + i % kChunkCols];
    }
    const float qscale = 1.0f / sqrtf(static_cast<float>(D));
    // Chunk-row products: thread (t = tid / 4) computes row t, columns
    // cq .. cq + 3 of the block's 16. State update: element e = tid,
    // tid + 256, ... of the D x 16 block (row e / 16, column e % 16).
    const uint32_t t = tid / 4, cq = (tid % 4) * 4;
    const uint32_t nchunks = (tokens + kChunk - 1) / kChunk;
    for (uint32_t c = 0; c < nchunks; ++c) {
        const uint32_t t0 = c * kChunk, len = min(kChunk, tokens - t0);
        const float* T = tp + (static_cast<size_t>(c) * value_heads + h) * 2 * kChunk * kChunk;
        const float* P = T + kChunk * kChunk;
        __syncthreads();  // the previous chunk's reads of Ks / Qs / Ds are done
        chunk_rows<D, VEC>(k, ldqk, kh * D, t0, len, Ks);
        chunk_rows<D, VEC>(q, ldqk, kh * D, t0, len, Qs);
        {
            float4 tr[4], pr[4];
#pragma unroll
            for (uint32_t n = 0; n < 4; ++n) {
                tr[n] = reinterpret_cast<const float4*>(T)[tid + 256 * n];
                pr[n] = reinterpret_cast<const float4*>(P)[tid + 256 * n];
            }
#pragma unroll
            for (uint32_t n = 0; n < 4; ++n) {
                const uint32_t i = 4 * (tid + 256 * n), r = i / kChunk, c4 = i % kChunk;
                Ts[r][c4] = tr[n].x, Ts[r][c4 + 1] = tr[n].y, Ts[r][c4 + 2] = tr[n].z, Ts[r][c4 + 3] = tr[n].w;
                Ps[r][c4] = pr[n].x, Ps[r][c4 + 1] = pr[n].y, Ps[r][c4 + 2] = pr[n].z, Ps[r][c4 + 3] = pr[n].w;
            }
        }
        chunk_gates(decay, beta, value_heads, h, t0, len, G, B);
        __syncthreads();
        if (tid < kChunk) E[tid] = expf(G[kChunk - 1] - G[tid]);
        // X1 = K S0, Y1 = Q S0 for row t, columns cq .. cq + 3.
        float x1[4] = {}, y1[4] = {};
        for (uint32_t d = 0; d < D; ++d) {
            const float kt = Ks[t][d], qt = Qs[t][d];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x1[j] = fmaf(kt, Ss[d][cq + j], x1[j]);
                y1[j] = fmaf(qt, Ss[d][cq + j], y1[j]);
            }
        }
        const float eg = expf(G[t]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float vv = t < len ? v[static_cast<size_t>(t0 + t) * ldv + h * D + col0 + cq + j] : 0.0f;
            Rs[t][cq + j] = B[t] * (vv - eg * x1[j]);
        }
        __syncthreads();
        // Delta = T R (T unit lower triangular).
        float dl[4] = {};
        for (uint32_t i = 0; i <= t; ++i) {
            const float ti = Ts[t][i];
#pragma unroll
            for (int j = 0; j < 4; ++j) dl[j] = fmaf(ti, Rs[i][cq + j], dl[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) Ds[t][cq + j] = dl[j];
        __syncthreads();
        // Outputs, then the state update (every read of the old state is done).
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = eg * y1[j];
        for (uint32_t i = 0; i <= t; ++i) {
            const float pi = Ps[t][i];
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = fmaf(pi, Ds[i][cq + j], o[j]);
        }
        if (t < len) {
#pragma unroll
            for (int j = 0; j < 4; ++j) out[static_cast<size_t>(t0 + t) * ldo + h * D + col0 + cq + j] = o[j] * qscale;
        }
        const float keep = expf(G[kChunk - 1]);
        for (uint32_t e = tid; e < D * kChunkCols; e += 256) {
            const uint32_t r = e / kChunkCols, j = e % kChunkCols;
            float acc = 0.0f;
            for (uint32_t i = 0; i < kChunk; ++i) acc = fmaf(Ks[i][r] * E[i], Ds[i][j], acc);
            Ss[r][j] = fmaf(keep, Ss[r][j], acc);
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < D * kChunkCols; i += 256) {
        S[static_cast<size_t>(i / kChunkCols) * D + col0 + i % kChunkCols] = Ss[i / kChunkCols][i % kChunkCols];
    }
}

// Fused decode/prefill forms of the DeltaNet pieces above.
//
// Causal conv + SiLU + the L2 head norm in one pass: block `seg` owns the D
// channels of one head segment ([seg D, seg D + D)), one thread per channel,
// all tokens in order (history read first, written last); segments below
// norm_channels (the Q and K heads) are L2-normalised per token with a
// block-wide sum of squares. Same expressions as conv1d_silu_kernel and
// l2norm_heads_kernel.
template <uint32_t D>
__global__ __launch_bounds__(D) void conv_l2norm_kernel(const float* __restrict__ x, uint32_t ldx,
                                                        float* __restrict__ history, const float* __restrict__ w,
                                                        float* __restrict__ out, uint32_t ldo, uint32_t tokens,
                                                        uint32_t channels, uint32_t ksize, uint32_t norm_channels,
                                                        float eps) {
    constexpr uint32_t W = D / 64;
    const uint32_t c = blockIdx.x * D + threadIdx.x;
    const bool norm = blockIdx.x * D < norm_channels;  // uniform per block
    const uint32_t hr = ksize - 1;
    __shared__ float red[W];
    float win[kMaxConv];
    float taps[kMaxConv];
    for (uint32_t i = 0; i < ksize; ++i) taps[i] = w[static_cast<size_t>(c) * ksize + i];
    for (uint32_t i = 0; i < hr; ++i) win[i] = history[static_cast<size_t>(i) * channels + c];
    for (uint32_t t = 0; t < tokens; ++t) {
        win[hr] = x[static_cast<size_t>(t) * ldx + c];
        float acc = 0.0f;
        for (uint32_t i = 0; i < ksize; ++i) acc += win[i] * taps[i];
        float v = acc * sigmoid_ref(acc);
        if (norm) {
            const float ss = wave_sum(v * v);
            if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
            __syncthreads();
            float tot = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < W; ++i) tot += red[i];
            v = v * (1.0f / sqrtf(tot + eps));
            __syncthreads();  // red[] reused by the next token
        }
        out[static_cast<size_t>(t) * ldo + c] = v;
        for (uint32_t i = 0; i < hr; ++i) win[i] = win[i + 1];
    }
    for (uint32_t i = 0; i < hr; ++i) history[static_cast<size_t>(i) * channels + c] = win[i];
}

// Gated DeltaNet scan with its gates and the gated RMSNorm fused. Block =
// value head h (all D columns), 256 threads: thread (col = tid % D,
// rg = tid / D) holds rows [rg NPR, rg NPR + NPR) of column col of S_h.
// Per token: decay = exp(softplus(alpha + dt_bias) a), beta = sigmoid(beta_raw)
// (gdn_gates_kernel's expressions), the recurrence of gdn_scan_kernel, then
// y = rmsnorm(o) * gamma * silu(z) over the head (gated_rmsnorm_kernel) and
// its XGroup form. The state is read and written once per call.
template <uint32_t D>
__global__ __launch_bounds__(256) void gdn_scan_gated_kernel(
    const float* __restrict__ q, const float* __restrict__ k, uint32_t ldqk, const float* __restrict__ v,
    uint32_t ldv, const float* __restrict__ alpha, const float* __restrict__ beta_raw, uint32_t ld_ab,
    const float* __restrict__ dt_bias, const float* __restrict__ a, float* __restrict__ state,
    const float* __restrict__ z, uint32_t ldz, const float* __restrict__ gamma, float* __restrict__ y,
    XGroup* __restrict__ yq, uint32_t ldy, uint32_t tokens, uint32_t key_heads, float eps) {
    constexpr uint32_t RG = 256 / D, NPR = D / RG;
    const uint32_t h = blockIdx.x;
    const uint32_t col = threadIdx.x % D, rg = threadIdx.x / D;
    const uint32_t kh = h % key_heads;
    float* S = state + static_cast<size_t>(h) * D * D;
    float s[NPR];
#pragma unroll
    for (uint32_t i = 0; i < NPR; ++i) s[i] = S[static_cast<size_t>(rg * NPR + i) * D + col];
    __shared__ float ks[D], qs[D];
    __shared__ float part[RG][D];
    __shared__ float red[D / 64];
    __shared__ __align__(16) float vals[D];
    const float qscale = 1.0f / sqrtf(static_cast<float>(D));
    const float dtb = dt_bias[h], ah = a[h], gam = gamma[col];
    for (uint32_t t = 0; t < tokens; ++t) {
        for (uint32_t i = threadIdx.x; i < D; i += 256) {
            ks[i] = k[static_cast<size_t>(t) * ldqk + kh * D + i];
            qs[i] = q[static_cast<size_t>(t) * ldqk + kh * D + i];
        }
        const float g = expf(softplus_ref(alpha[static_cast<size_t>(t) * ld_ab + h] + dtb) * ah);
        const float b = sigmoid_ref(beta_raw[static_cast<size_t>(t) * ld_ab + h]);
        const float vv = v[static_cast<size_t>(t) * ldv + h * D + col];
        __syncthreads();
        float pp = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < NPR; ++i) {
            s[i] *= g;
            pp += s[i] * ks[rg * NPR + i];
        }
        part[rg][col] = pp;
        __syncthreads();
        float pred = 0.0f;
#pragma unroll
        for (uint32_t r = 0; r < RG; ++r) pred += part[r][col];
        const float delta = b * (vv - pred);
        float op = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < NPR; ++i) {
            s[i] += ks[rg * NPR + i] * delta;
            op += s[i] * qs[rg * NPR + i];
        }
        __syncthreads();  // everyone has read part[] (pred) before it is reused
        part[rg][col] = op;
        __syncthreads();
        float o = 0.0f;
#pragma unroll
        for (uint32_t r = 0; r < RG; ++r) o += part[r][col];
        o *= qscale;
        // Gated RMSNorm over the head's D outputs (threads rg == 0 hold them).
        if (rg == 0) {
            const float ss = wave_sum(o * o);
            if ((col & 63) == 0) red[col >> 6] = ss;
        }
        __syncthreads();
        if (rg == 0) {
            float tot = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < D / 64; ++i) tot += red[i];
            const float inv = 1.0f / sqrtf(tot / static_cast<float>(D) + eps);
            const float zz = z[static_cast<size_t>(t) * ldz + h * D + col];
            const float yv = o * inv * gam * (zz * sigmoid_ref(zz));
            y[static_cast<size_t>(t) * ldy + h * D + col] = yv;
            vals[col] = yv;
        }
        __syncthreads();
        if (yq && threadIdx.x < D / 16) {
            xgroup_encode_from(vals + 16 * threadIdx.x,
                               yq + static_cast<size_t>(t) * (ldy / 16) + static_cast<size_t>(h) * (D / 16) +
                                   threadIdx.x);
        }
        __syncthreads();  // ks/qs/part/red/vals reused by the next token
    }
#pragma unroll
    for (uint32_t i = 0; i < NPR; ++i) S[static_cast<size_t>(rg * NPR + i) * D + col] = s[i];
}

// One decode token of a Gated DeltaNet layer after its projections, block h
// = value head h (256 threads). qkv is the token's convolved [Q (G D) | K
// (G D) | V (Hv D)] row (the conv + SiLU ran in the projection's epilogue),
// z the gate row. The block also makes its own two gate inputs: with x the
// layer's raw input row and x_gamma its RMSNorm gain, alpha_h and beta_h are
// the dots of rows h and Hv + h of the F32 projection ab_w ([2 Hv, hidden])
// with rmsnorm(x) * x_gamma (double sum of squares as in the RMSNorm
// kernel). Then the L2 norms of Q and K head kh = h % G (wave sums in order,
// as conv_l2norm_kernel), and gdn_scan_gated_kernel's gates, recurrence and
// gated RMSNorm. All loads are issued at the start: state, the head's Q, K,
// V and z values, x, its gain and the two projection rows.
constexpr uint32_t kGdnDecodeMaxHidden = 4096;

template <uint32_t D>
__global__ __launch_bounds__(256) void gdn_decode_kernel(
    const float* __restrict__ qkv, const float* __restrict__ x, const float* __restrict__ x_gamma,
    const float* __restrict__ ab_w, uint32_t hidden, const float* __restrict__ dt_bias, const float* __restrict__ a,
    float* __restrict__ state, const float* __restrict__ z, const float* __restrict__ gamma, float* __restrict__ y,
    XGroup* __restrict__ yq, uint32_t value_heads, uint32_t key_heads, float eps) {
    constexpr uint32_t RG = 256 / D, NPR = D / RG;
    constexpr uint32_t NX = kGdnDecodeMaxHidden / 256;
    const uint32_t h = blockIdx.x, tid = threadIdx.x;
    const uint32_t col = tid % D, rg = tid / D, wave = tid >> 6, lane = tid & 63;
    const uint32_t G = key_heads, kh = h % G;
    float* S = state + static_cast<size_t>(h) * D * D;
    float s[NPR];
#pragma unroll
    for (uint32_t i = 0; i < NPR; ++i) s[i] = S[static_cast<size_t>(rg * NPR + i) * D + col];
    const float qk = tid < 2 * D ? qkv[(tid < D ? kh : G + kh) * D + tid % D] : 0.0f;
    const float vv = qkv[(2 * G + h) * D + col];
    const float zz = z[static_cast<size_t>(h) * D + col];
    const float dtb = dt_bias[h], ah = a[h], gam = gamma[col];
    const float* wa = ab_w + static_cast<size_t>(h) * hidden;
    const float* wb = ab_w + static_cast<size_t>(value_heads + h) * hidden;
    float xv[NX], gv[NX], av[NX], bv[NX];
#pragma unroll
    for (uint32_t i = 0; i < NX; ++i) {
        const uint32_t e = tid + 256 * i;
        const bool ok = e < hidden;
        xv[i] = ok ? x[e] : 0.0f;
        gv[i] = ok ? x_gamma[e] : 0.0f;
        av[i] = ok ? wa[e] : 0.0f;
        bv[i] = ok ? wb[e] : 0.0f;
    }
    __shared__ double red_d[4];
    __shared__ float red_f[3][4];
    // Input RMSNorm and the two gate dots.
    double ss = 0.0;
#pragma unroll
    for (uint32_t i = 0; i < NX; ++i) ss += static_cast<double>(xv[i]) * xv[i];
    ss = wave_sum_d(ss);
    // Q / K head sums of squares (waves [0, D / 64) hold Q, the next D / 64 K).
    const float qss = wave_sum(qk * qk);
    if (lane == 0) {
        red_d[wave] = ss;
        red_f[0][wave] = qss;
    }
    __syncthreads();
    const double tot = (red_d[0] + red_d[1]) + (red_d[2] + red_d[3]);
    const float inv = 1.0f / sqrtf(static_cast<float>(tot / static_cast<double>(hidden)) + eps);
    float da = 0.0f, db = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < NX; ++i) {
        const float xn = xv[i] * (inv * gv[i]);
        da = fmaf(av[i], xn, da);
        db = fmaf(bv[i], xn, db);
    }
    da = wave_sum(da);
    db = wave_sum(db);
    if (lane == 0) {
        red_f[1][wave] = da;
        red_f[2][wave] = db;
    }
    __shared__ float ks[D], qs[D];
    if (tid < 2 * D) {
        const uint32_t seg = tid / D;
        float t = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < D / 64; ++j) t += red_f[0][seg * (D / 64) + j];
        const float v = qk * (1.0f / sqrtf(t + eps));
        if (seg == 0) {
            qs[tid] = v;
        } else {
            ks[tid - D] = v;
        }
    }
    __syncthreads();
    const float alpha = (red_f[1][0] + red_f[1][1]) + (red_f[1][2] + red_f[1][3]);
    const float beta_raw = (red_f[2][0] + red_f[2][1]) + (red_f[2][2] + red_f[2][3]);

    // gdn_scan_gated_kernel's token step.
    __shared__ float part[RG][D];
    __shared__ float red[D / 64];
    __shared__ __align__(16) float vals[D];
    const float qscale = 1.0f / sqrtf(static_cast<float>(D));
    const float g = expf(softplus_ref(alpha + dtb) * ah);
    const float b = sigmoid_ref(beta_raw);
    float pp = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < NPR; ++i) {
        s[i] *= g;
        pp += s[i] * ks[rg * NPR + i];
    }
    part[rg][col] = pp;
    __syncthreads();
    float pred = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < RG; ++q) pred += part[q][col];
    const float delta = b * (vv - pred);
    float op = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < NPR; ++i) {
        s[i] += ks[rg * NPR + i] * delta;
        op += s[i] * qs[rg * NPR + i];
    }
#pragma unroll
    for (uint32_t i = 0; i < NPR; ++i) S[static_cast<size_t>(rg * NPR + i) * D + col] = s[i];
    __syncthreads();  // everyone has read part[] (pred) before it is reused
    part[rg][col] = op;
    __syncthreads();
    float o = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < RG; ++q) o += part[q][col];
    o *= qscale;
    if (rg == 0) {
        const float oss = wave_sum(o * o);
        if ((col & 63) == 0) red[col >> 6] = oss;
    }
    __syncthreads();
    if (rg == 0) {
        float t = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < D / 64; ++i) t += red[i];
        const float on = 1.0f / sqrtf(t / static_cast<float>(D) + eps);
        const float yv = o * on * gam * (zz * sigmoid_ref(zz));
        y[static_cast<size_t>(h) * D + col] = yv;
        vals[col] = yv;
    }
    if (yq) {
        __syncthreads();
        if (tid < D / 16) xgroup_encode_from(vals + 16 * tid, yq + static_cast<size_t>(h) * (D / 16) + tid);
    }
}

// y = rmsnorm(o_head) * gamma * silu(z) per (row, value head); FP32 sum of
// squares like the reference's per-head norm; yq (optional) the XGroup form
// of y.
__global__ __launch_bounds__(64) void gated_rmsnorm_kernel(const float* __restrict__ o, uint32_t ldo,
                                                          const float* __restrict__ gamma,
                                                          const float* __restrict__ z, uint32_t ldz,
                                                          float* __restrict__ y, XGroup* __restrict__ yq,
                                                          uint32_t ldy, uint32_t d, float eps) {
    const uint32_t t = blockIdx.x, h = blockIdx.y;
    const float* ov = o + static_cast<size_t>(t) * ldo + static_cast<size_t>(h) * d;
    const float* zv = z + static_cast<size_t>(t) * ldz + static_cast<size_t>(h) * d;
    float* yv = y + static_cast<size_t>(t) * ldy + static_cast<size_t>(h) * d;
    __shared__ __align__(16) float vals[256];
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < d; i += 64) ss += ov[i] * ov[i];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
    for (uint32_t i = threadIdx.x; i < d; i += 64) {
        const float zz = zv[i];
        const float v = ov[i] * inv * gamma[i] * (zz * sigmoid_ref(zz));
        yv[i] = v;
        vals[i] = v;
    }
    if (yq) {
        __syncthreads();
        const uint32_t groups = d / 16;
        for (uint32_t g = threadIdx.x; g < groups; g += 64) {
            xgroup_encode_from(vals + 16 * g, yq + static_cast<size_t>(t) * (ldy / 16) + static_cast<size_t>(h) * groups + g);
        }
    }
}

// ------------------------------------------------------------ full attention
// Block (row t, head h), one wave. h < hq: the interleaved [Q_h | gate_h]
// pair of `mixed` -> RMSNorm(Q_h) * q_gamma into qkv's Q part, gate_h into
// `gate`. h >= hq: KV head j = h - hq of `kv` ([K | V] rows) ->
// RMSNorm(K_j) * k_gamma into qkv's K part and V_j copied into its V part.
__global__ __launch_bounds__(64) void split_qgate_norm_kernel(const float* __restrict__ mixed, uint32_t ldm,
                                                             const float* __restrict__ kv, uint32_t ldkv,
                                                             const float* __restrict__ q_gamma,
                                                             const float* __restrict__ k_gamma,
                                                             float* __restrict__ qkv, uint32_t ldqkv,
                                                             float* __restrict__ gate, uint32_t ldg, uint32_t hq,
                                                             uint32_t hkv, uint32_t d, float eps) {
    const uint32_t t = blockIdx.x, h = blockIdx.y;
    const float* src;
    const float* gamma;
    float* dst;
    if (h < hq) {
        src = mixed + static_cast<size_t>(t) * ldm + static_cast<size_t>(h) * 2 * d;
        gamma = q_gamma;
        dst = qkv + static_cast<size_t>(t) * ldqkv + static_cast<size_t>(h) * d;
        float* g = gate + static_cast<size_t>(t) * ldg + static_cast<size_t>(h) * d;
        for (uint32_t i = threadIdx.x; i < d; i += 64) g[i] = src[d + i];
    } else {
        const uint32_t j = h - hq;
        src = kv + static_cast<size_t>(t) * ldkv + static_cast<size_t>(j) * d;
        gamma = k_gamma;
        dst = qkv + static_cast<size_t>(t) * ldqkv + static_cast<size_t>(hq + j) * d;
        const float* vs = kv + static_cast<size_t>(t) * ldkv + static_cast<size_t>(hkv + j) * d;
        float* vd = qkv + static_cast<size_t>(t) * ldqkv + static_cast<size_t>(hq + hkv + j) * d;
        for (uint32_t i = threadIdx.x; i < d; i += 64) vd[i] = vs[i];
    }
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < d; i += 64) ss += src[i] * src[i];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
    for (uint32_t i = threadIdx.x; i < d; i += 64) dst[i] = src[i] * inv * gamma[i];
}

// y = a * sigmoid(g) per element, per-16 sums (optional) for the next GEMV.
__global__ void gate_mul_kernel(const float* __restrict__ a, const float* __restrict__ g, float* __restrict__ y,
                                XGroup* __restrict__ yq, size_t n16) {
    const size_t grp = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (grp >= n16) return;
    float v[16];
#pragma unroll
    for (uint32_t i = 0; i < 16; ++i) {
        const size_t idx = 16 * grp + i;
        v[i] = a[idx] * sigmoid_ref(g[idx]);
        y[idx] = v[i];
    }
    if (yq) xgroup_encode(v, yq + grp);
}

uint32_t blocks_for(size_t n, uint32_t threads) { return static_cast<uint32_t>((n + threads - 1) / threads); }

int launched() { return hipGetLastError() == hipSuccess ? kOk : kRuntimeError; }

}  // namespace

int launch_router_topk(const float* logits, size_t ld, size_t tokens, size_t experts, size_t k, int32_t* ids,
                       float* weights, hipStream_t stream) {
    if (!logits || !ids || !weights || tokens == 0 || experts == 0 || k == 0 || k > 8 || k > experts ||
        ld < experts) {
        return kInvalidArgument;
    }
    if (experts > kMaxExperts || tokens > 0x7fffffffull || ld > 0xffffffffull) return kLengthError;
    auto kernel = experts <= 256 ? router_topk_kernel<4> : experts <= 512 ? router_topk_kernel<8>
                                                                           : router_topk_kernel<kMaxExperts / 64>;
    HIPLLM_LAUNCH(kernel, dim3(static_cast<uint32_t>(tokens)), dim3(64), 0, stream, logits,
                       static_cast<uint32_t>(ld), static_cast<uint32_t>(experts), static_cast<uint32_t>(k), ids,
                       weights);
    return launched();
}

namespace {
// K split of the FP32 matmul: enough blocks for the GPU's 256 CUs, at least
// 128 k per split, at most 16 splits.
size_t matmul_splits(size_t m, size_t n, size_t k) {
    const size_t tiles = ((m + kMmTile - 1) / kMmTile) * ((n + kMmTile - 1) / kMmTile);
    size_t s = tiles >= 256 ? 1 : (256 + tiles - 1) / tiles;
    s = std::min<size_t>(s, std::min<size_t>(16, (k + kMmK - 1) / kMmK));
    const size_t kc = ((k + s - 1) / s + kMmK - 1) / kMmK * kMmK;
    return (k + kc - 1) / kc;
}
}  // namespace

size_t matmul_f32_scratch_floats(size_t m, size_t n, size_t k) {
    const size_t s = matmul_splits(m, n, k);
    return s > 1 ? s * m * n : 0;
}

int launch_matmul_f32(const float* x, size_t ldx, const float* w, size_t ldw, float* y, size_t ldy, size_t m, size_t n,
                      size_t k, float* scratch, size_t scratch_floats, hipStream_t stream) {
    if (!x || !w || !y || m == 0 || n == 0 || k == 0 || ldx < k || ldw < k || ldy < n) return kInvalidArgument;
    if (ldx > 0xffffffffull || ldw > 0xffffffffull || ldy > 0xffffffffull || k > 0xffffffffull ||
        (m + kMmTile - 1) / kMmTile > 65535 || (n + kMmTile - 1) / kMmTile > 0x7fffffffull || m * n > 0xffffffffull) {
        return kLengthError;
    }
    size_t s = matmul_splits(m, n, k);
    if (s > 1 && (!scratch || scratch_floats < s * m * n)) s = 1;  // no room for the partial sums: unsplit
    const size_t kc = s > 1 ? ((k + s - 1) / s + kMmK - 1) / kMmK * kMmK : k;
    const dim3 grid(static_cast<uint32_t>((n + kMmTile - 1) / kMmTile),
                    static_cast<uint32_t>((m + kMmTile - 1) / kMmTile), static_cast<uint32_t>(s));
    HIPLLM_LAUNCH(matmul_f32_kernel, grid, dim3(256), 0, stream, x, static_cast<uint32_t>(ldx), w,
                       static_cast<uint32_t>(ldw), y, static_cast<uint32_t>(ldy), static_cast<uint32_t>(m),
                       static_cast<uint32_t>(n), static_cast<uint32_t>(k), static_cast<uint32_t>(kc),
                       s > 1 ? scratch : nullptr);
    if (s > 1) {
        HIPLLM_LAUNCH(matmul_reduce_kernel, dim3(blocks_for(m * n, 256)), dim3(256), 0, stream, scratch, y,
                           static_cast<uint32_t>(ldy), static_cast<uint32_t>(m), static_cast<uint32_t>(n),
                           static_cast<uint32_t>(s));
    }
    return launched();
}

size_t route_groups_max(size_t n, size_t experts, size_t vmax) {
    return vmax == 0 ? 0 : (n + vmax - 1) / vmax + (experts < n ? experts : n);
}

int launch_route_groups(const int32_t* ids, size_t n, size_t experts, size_t vmax, int32_t* order, int32_t* groups,
                        uint32_t* ngroups, hipStream_t stream) {
    if (!ids || !order || !groups || !ngroups || n == 0 || experts == 0 || vmax == 0) return kInvalidArgument;
    if (n > kRouteGroupsMax || experts > kMaxExperts || vmax > 0xffffu) return kLengthError;
    HIPLLM_LAUNCH(route_groups_kernel, dim3(1), dim3(1024), 0, stream, ids, static_cast<uint32_t>(n),
                       static_cast<uint32_t>(experts), static_cast<uint32_t>(vmax), order, groups, ngroups);
    return launched();
}

int launch_moe_combine_norm(const float* residual, const float* down, const float* w, const float* shared,
                            const float* sgate, size_t ld_sgate, float* out, const float* gamma, float* norm,
                            XGroup* normq, size_t tokens, size_t h, size_t k, float eps, hipStream_t stream) {
    if (!residual || !down || !w || !out || !gamma || !norm || tokens == 0 || h == 0 || k == 0 ||
        (shared && (!sgate || !ld_sgate)) || !(eps > 0.0f) ||
        (normq && (h % 16 != 0 || reinterpret_cast<uintptr_t>(normq) % 16 != 0))) {
        return kInvalidArgument;
    }
    // The norm's vector path reads and writes 16-byte aligned rows.
    if (h % 4 == 0) {
        for (const void* p : {static_cast<const void*>(out), static_cast<const void*>(gamma),
                              static_cast<const void*>(norm), static_cast<const void*>(residual),
                              static_cast<const void*>(down), static_cast<const void*>(shared)}) {
            if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return kInvalidArgument;  // nullptr passes
        }
    }
    if (tokens > 0x7fffffffull || ld_sgate > 0xffffffffull || h > 0x7fffffffull / 4) return kLengthError;
    HIPLLM_LAUNCH(moe_combine_norm_kernel, dim3(static_cast<uint32_t>(tokens)), dim3(256), 0, stream, residual,
                       down, w, shared, sgate, static_cast<uint32_t>(ld_sgate), out, gamma, norm, normq,
                       static_cast<uint32_t>(h), static_cast<uint32_t>(k), eps);
    return launched();
}

int launch_moe_combine(const float* residual, const float* down, const float* w, const float* shared,
                       const float* sgate, size_t ld_sgate, float* out, size_t tokens, size_t h, size_t k,
                       hipStream_t stream) {
    if (!residual || !down || !w || !out || tokens == 0 || h == 0 || k == 0 || (shared && (!sgate || !ld_sgate))) {
        return kInvalidArgument;
    }
    if (tokens * h > 0x7fffffffull * 256ull || ld_sgate > 0xffffffffull || h > 0xffffffffull) return kLengthError;
    HIPLLM_LAUNCH(moe_combine_kernel, dim3(blocks_for(tokens * h, 256)), dim3(256), 0, stream, residual, down,
                       w, shared, sgate, static_cast<uint32_t>(ld_sgate), out, static_cast<uint32_t>(tokens),
                       static_cast<uint32_t>(h), static_cast<uint32_t>(k));
    return launched();
}

int launch_gdn_gates(const float* alpha, const float* beta_raw, size_t ld, const float* dt_bias, const float* a,
                     float* decay, float* beta, size_t tokens, size_t heads, hipStream_t stream) {
    if (!alpha || !beta_raw || !dt_bias || !a || !decay || !beta || tokens == 0 || heads == 0 || ld < heads) {
        return kInvalidArgument;
    }
    if (tokens * heads > 0x7fffffffull) return kLengthError;
    HIPLLM_LAUNCH(gdn_gates_kernel, dim3(blocks_for(tokens * heads, 256)), dim3(256), 0, stream, alpha,
                       beta_raw, static_cast<uint32_t>(ld), dt_bias, a, decay, beta, static_cast<uint32_t>(tokens),
                       static_cast<uint32_t>(heads));
    return launched();
}

int launch_conv1d_silu(const float* x, size_t ldx, float* history, const float* w, float* out, size_t ldo,
                       size_t tokens, size_t channels, size_t ksize, hipStream_t stream) {
    if (!x || !history || !w || !out || tokens == 0 || channels == 0 || ksize < 2 || ksize > kMaxConv ||
        ldx < channels || ldo < channels) {
        return kInvalidArgument;
    }
    if (x == out) return kInvalidArgument;
    if (channels > 0x7fffffffull || (tokens + kConvChunk - 1) / kConvChunk > 65535) return kLengthError;
    const dim3 grid(static_cast<uint32_t>((channels + 63) / 64),
                    static_cast<uint32_t>((tokens + kConvChunk - 1) / kConvChunk));
    HIPLLM_LAUNCH(conv1d_silu_kernel, grid, dim3(256), 0, stream, x, static_cast<uint32_t>(ldx), history, w, out,
                       static_cast<uint32_t>(ldo), static_cast<uint32_t>(tokens), static_cast<uint32_t>(channels),
                       static_cast<uint32_t>(ksize));
    return launched();
}

int launch_l2norm_heads(float* x, size_t ld, size_t tokens, size_t heads, size_t d, float eps, hipStream_t stream) {
    if (!x || tokens == 0 || heads == 0 || d == 0 || ld < heads * d || !(eps >= 0.0f)) return kInvalidArgument;
    if (tokens > 0x7fffffffull || heads > 65535) return kLengthError;
    HIPLLM_LAUNCH(l2norm_heads_kernel, dim3(static_cast<uint32_t>(tokens), static_cast<uint32_t>(heads)),
                       dim3(64), 0, stream, x, static_cast<uint32_t>(ld), static_cast<uint32_t>(d), eps);
    return launched();
}

int launch_gdn_scan(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv, const float* decay,
                    const float* beta, float* state, float* out, size_t ldo, size_t tokens, size_t value_heads,
                    size_t key_heads, size_t d, hipStream_t stream) {
    if (!q || !k || !v || !decay || !beta || !state || !out || tokens == 0 || value_heads == 0 || key_heads == 0 ||
        value_heads % key_heads != 0) {
        return kInvalidArgument;
    }
    if (d != 64 && d != 128) return kInvalidArgument;  // state size 64 or 128
    if (ldqk < key_heads * d || ldv < value_heads * d || ldo < value_heads * d) return kInvalidArgument;
    if (tokens > 0x7fffffffull || value_heads > 0x7fffffffull) return kLengthError;
    if (value_heads > 0x7fffffffull / d) return kLengthError;
    const dim3 grid(static_cast<uint32_t>(value_heads * (d / 4)));
    const uint32_t T = static_cast<uint32_t>(tokens), Hv = static_cast<uint32_t>(value_heads),
                   Hk = static_cast<uint32_t>(key_heads);
    // Whole float4 loads of k and q when their rows start on 16 bytes.
    const bool vec = reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                     ldqk % 4 == 0;
    const uint32_t lq = static_cast<uint32_t>(ldqk), lv = static_cast<uint32_t>(ldv), lo = static_cast<uint32_t>(ldo);
    if (d == 64 && vec) {
        HIPLLM_LAUNCH((gdn_scan_kernel<64, true>), grid, dim3(64), 0, stream, q, k, lq, v, lv, decay, beta, state,
                           out, lo, T, Hv, Hk);
    } else if (d == 64) {
        HIPLLM_LAUNCH((gdn_scan_kernel<64, false>), grid, dim3(64), 0, stream, q, k, lq, v, lv, decay, beta, state,
                           out, lo, T, Hv, Hk);
    } else if (d == 128 && vec) {
        HIPLLM_LAUNCH((gdn_scan_kernel<128, true>), grid, dim3(64), 0, stream, q, k, lq, v, lv, decay, beta,
                           state, out, lo, T, Hv, Hk);
    } else if (d == 128) {
        HIPLLM_LAUNCH((gdn_scan_kernel<128, false>), grid, dim3(64), 0, stream, q, k, lq, v, lv, decay, beta,
                           state, out, lo, T, Hv, Hk);
    } else {
        return kInvalidArgument;  // state size 64 or 128
    }
    return launched();
}

size_t gdn_chunk_scratch_floats(size_t tokens, size_t value_heads) {
    return (tokens + kChunk - 1) / kChunk * value_heads * 2 * kChunk * kChunk;
}

int launch_gdn_scan_chunked(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv,
                            const float* decay, const float* beta, float* state, float* out, size_t ldo,
                            size_t tokens, size_t value_heads, size_t key_heads, size_t d, float* scratch,
                            size_t scratch_floats, hipStream_t stream) {
    if (!q || !k || !v || !decay || !beta || !state || !out || !scratch || tokens == 0 || value_heads == 0 ||
        key_heads == 0 || value_heads % key_heads != 0) {
        return kInvalidArgument;
    }
    if (d != 64 && d != 128) return kInvalidArgument;  // state size 64 or 128
    if (ldqk < key_heads * d || ldv < value_heads * d || ldo < value_heads * d) return kInvalidArgument;
    if (tokens > 0x7fffffffull || value_heads > 65535) return kLengthError;
    if (scratch_floats < gdn_chunk_scratch_floats(tokens, value_heads)) return kInvalidArgument;
    const uint32_t T = static_cast<uint32_t>(tokens), Hv = static_cast<uint32_t>(value_heads),
                   Hk = static_cast<uint32_t>(key_heads), chunks = (T + kChunk - 1) / kChunk;
    if (chunks > 65535) return kLengthError;
    const uint32_t lq = static_cast<uint32_t>(ldqk), lv = static_cast<uint32_t>(ldv), lo = static_cast<uint32_t>(ldo);
    // Whole float4 loads of k and q when their rows start on 16 bytes; the
    // scratch (T and P of every chunk) is read as float4.
    if (reinterpret_cast<uintptr_t>(scratch) % 16 != 0) return kInvalidArgument;
    const bool vec = reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                     ldqk % 4 == 0;
    auto run = [&](auto dc, auto vc) {
        constexpr uint32_t DD = decltype(dc)::value;
        constexpr bool V = decltype(vc)::value;
        HIPLLM_LAUNCH((gdn_chunk_prep_kernel<DD, V>), dim3(Hv, chunks), dim3(256), 0, stream, q, k, lq, decay,
                           beta, scratch, T, Hv, Hk);
        HIPLLM_LAUNCH((gdn_chunk_scan_kernel<DD, V>), dim3(Hv * (DD / kChunkCols)), dim3(256), 0, stream, q, k,
                           lq, v, lv, decay, beta, scratch, state, out, lo, T, Hv, Hk);
    };
    using D128 = std::integral_constant<uint32_t, 128>;
    using D64 = std::integral_constant<uint32_t, 64>;
    if (d == 128 && vec) run(D128{}, std::true_type{});
    else if (d == 128) run(D128{}, std::false_type{});
    else if (vec) run(D64{}, std::true_type{});
    else run(D64{}, std::false_type{});
    return launched();
}

int launch_gated_rmsnorm(const float* o, size_t ldo, const float* gamma, const float* z, size_t ldz, float* y,
                         XGroup* yq, size_t ldy, size_t tokens, size_t heads, size_t d, float eps,
                         hipStream_t stream) {
    if (!o || !gamma || !z || !y || tokens == 0 || heads == 0 || d == 0 || d > 256 || ldo < heads * d ||
        ldz < heads * d || ldy < heads * d || !(eps > 0.0f)) {
        return kInvalidArgument;
    }
    if (yq && (d % 16 != 0 || ldy % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0)) return kInvalidArgument;
    if (tokens > 0x7fffffffull || heads > 65535) return kLengthError;
    HIPLLM_LAUNCH(gated_rmsnorm_kernel, dim3(static_cast<uint32_t>(tokens), static_cast<uint32_t>(heads)),
                       dim3(64), 0, stream, o, static_cast<uint32_t>(ldo), gamma, z, static_cast<uint32_t>(ldz), y,
                       yq, static_cast<uint32_t>(ldy), static_cast<uint32_t>(d), eps);
    return launched();
}

int launch_conv_l2norm(const float* x, size_t ldx, float* history, const float* w, float* out, size_t ldo,
                       size_t tokens, size_t channels, size_t ksize, size_t norm_channels, size_t d, float eps,
                       hipStream_t stream) {
    if (!x || !history || !w || !out || tokens == 0 || channels == 0 || ksize < 2 || ksize > kMaxConv ||
        ldx < channels || ldo < channels || x == out || !(eps >= 0.0f)) {
        return kInvalidArgument;
    }
    if ((d != 64 && d != 128) || channels % d != 0 || norm_channels % d != 0 || norm_channels > channels) {
        return kInvalidArgument;
    }
    if (channels > 0x7fffffffull || tokens > 0x7fffffffull) return kLengthError;
    const dim3 grid(static_cast<uint32_t>(channels / d));
    const uint32_t T = static_cast<uint32_t>(tokens), C = static_cast<uint32_t>(channels),
                   K = static_cast<uint32_t>(ksize), NC = static_cast<uint32_t>(norm_channels);
    if (d == 64) {
        HIPLLM_LAUNCH(conv_l2norm_kernel<64>, grid, dim3(64), 0, stream, x, static_cast<uint32_t>(ldx), history,
                           w, out, static_cast<uint32_t>(ldo), T, C, K, NC, eps);
    } else {
        HIPLLM_LAUNCH(conv_l2norm_kernel<128>, grid, dim3(128), 0, stream, x, static_cast<uint32_t>(ldx), history,
                           w, out, static_cast<uint32_t>(ldo), T, C, K, NC, eps);
    }
    return launched();
}

int launch_gdn_scan_gated(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv, const float* alpha,
                          const float* beta_raw, size_t ld_ab, const float* dt_bias, const float* a, float* state,
                          const float* z, size_t ldz, const float* gamma, float* y, XGroup* yq, size_t ldy,
                          size_t tokens, size_t value_heads, size_t key_heads, size_t d, float eps,
                          hipStream_t stream) {
    if (!q || !k || !v || !alpha || !beta_raw || !dt_bias || !a || !state || !z || !gamma || !y || tokens == 0 ||
        value_heads == 0 || key_heads == 0 || value_heads % key_heads != 0 || !(eps > 0.0f)) {
        return kInvalidArgument;
    }
    if (ldqk < key_heads * d || ldv < value_heads * d || ldz < value_heads * d || ldy < value_heads * d ||
        ld_ab < value_heads) {
        return kInvalidArgument;
    }
    if (yq && (ldy % 16 != 0 || reinterpret_cast<uintptr_t>(yq) % 16 != 0)) return kInvalidArgument;
    if (tokens > 0x7fffffffull || value_heads > 0x7fffffffull) return kLengthError;
    const dim3 grid(static_cast<uint32_t>(value_heads));
    const uint32_t T = static_cast<uint32_t>(tokens), Hk = static_cast<uint32_t>(key_heads);
    switch (d) {
    case 64:
        HIPLLM_LAUNCH(gdn_scan_gated_kernel<64>, grid, dim3(256), 0, stream, q, k, static_cast<uint32_t>(ldqk), v,
                           static_cast<uint32_t>(ldv), alpha, beta_raw, static_cast<uint32_t>(ld_ab), dt_bias, a,
                           state, z, static_cast<uint32_t>(ldz), gamma, y, yq, static_cast<uint32_t>(ldy), T, Hk, eps);
        break;
    case 128:
        HIPLLM_LAUNCH(gdn_scan_gated_kernel<128>, grid, dim3(256), 0, stream, q, k, static_cast<uint32_t>(ldqk), v,
                           static_cast<uint32_t>(ldv), alpha, beta_raw, static_cast<uint32_t>(ld_ab), dt_bias, a,
                           state, z, static_cast<uint32_t>(ldz), gamma, y, yq, static_cast<uint32_t>(ldy), T, Hk, eps);
        break;
    default:
        return kInvalidArgument;  // state size 64 or 128
    }
    return launched();
}

int launch_gdn_decode(const float* qkv, const float* x, const float* x_gamma, const float* ab_w, size_t hidden,
                      const float* dt_bias, const float* a, float* state, const float* z, const float* gamma, float* y,
                      XGroup* yq, size_t value_heads, size_t key_heads, size_t d, float eps, hipStream_t stream) {
    if (!qkv || !x || !x_gamma || !ab_w || !dt_bias || !a || !state || !z || !gamma || !y || key_heads == 0 ||
        value_heads == 0 || value_heads % key_heads != 0 || hidden == 0 || hidden > kGdnDecodeMaxHidden ||
        !(eps > 0.0f)) {
        return kInvalidArgument;
    }
    if (yq && reinterpret_cast<uintptr_t>(yq) % 16 != 0) return kInvalidArgument;
    if (value_heads > 65535) return kLengthError;
    const dim3 grid(static_cast<uint32_t>(value_heads));
    const uint32_t Hv = static_cast<uint32_t>(value_heads), Hk = static_cast<uint32_t>(key_heads),
                   Hd = static_cast<uint32_t>(hidden);
    switch (d) {
    case 64:
        HIPLLM_LAUNCH(gdn_decode_kernel<64>, grid, dim3(256), 0, stream, qkv, x, x_gamma, ab_w, Hd, dt_bias, a, state,
                      z, gamma, y, yq, Hv, Hk, eps);
        break;
    case 128:
        HIPLLM_LAUNCH(gdn_decode_kernel<128>, grid, dim3(256), 0, stream, qkv, x, x_gamma, ab_w, Hd, dt_bias, a,
                      state, z, gamma, y, yq, Hv, Hk, eps);
        break;
    default:
        return kInvalidArgument;  // state size 64 or 128
    }
    return launched();
}

int launch_split_qgate_norm(const float* mixed, size_t ldm, const float* kv, size_t ldkv, const float* q_gamma,
                            const float* k_gamma, float* qkv, size_t ldqkv, float* gate, size_t ldg, size_t tokens,
                            size_t hq, size_t hkv, size_t d, float eps, hipStream_t stream) {
    if (!mixed || !kv || !q_gamma || !k_gamma || !qkv || !gate || tokens == 0 || hq == 0 || hkv == 0 || d == 0 ||
        hq % hkv != 0 || !(eps > 0.0f)) {
        return kInvalidArgument;
    }
    if (ldm < 2 * hq * d || ldkv < 2 * hkv * d || ldqkv < (hq + 2 * hkv) * d || ldg < hq * d) return kInvalidArgument;
    if (tokens > 0x7fffffffull || hq + hkv > 65535) return kLengthError;
    HIPLLM_LAUNCH(split_qgate_norm_kernel, dim3(static_cast<uint32_t>(tokens), static_cast<uint32_t>(hq + hkv)),
                       dim3(64), 0, stream, mixed, static_cast<uint32_t>(ldm), kv, static_cast<uint32_t>(ldkv),
                       q_gamma, k_gamma, qkv, static_cast<uint32_t>(ldqkv), gate, static_cast<uint32_t>(ldg),
                       static_cast<uint32_t>(hq), static_cast<uint32_t>(hkv), static_cast<uint32_t>(d), eps);
    return launched();
}

int launch_gate_mul(const float* a, const float* g, float* y, XGroup* yq, size_t n, hipStream_t stream) {
    if (!a || !g || !y || n == 0 || n % 16 != 0) return kInvalidArgument;
    if (yq && reinterpret_cast<uintptr_t>(yq) % 16 != 0) return kInvalidArgument;
    const size_t n16 = n / 16;
    if (n16 > 0x7fffffffull) return kLengthError;
    HIPLLM_LAUNCH(gate_mul_kernel, dim3(blocks_for(n16, 256)), dim3(256), 0, stream, a, g, y, yq, n16);
    return launched();
}

}  // namespace hipllm
