/*
 * HipLLM C ABI (libhipllm.so): the drop-in boundary of the MI355X backend.
 *
 * Two layers:
 *  1. Kernel launchers. Caller-owned device pointers, a HIP stream passed as
 *     `void*` (hipStream_t; NULL = default stream), no allocation, return a
 *     status code. Each names the reference interface it replaces.
 *  2. A handle API that mirrors the reference backends' class contract
 *     (MetalLLM, metal_llm.h:20-52; CPULLM, cpu_llm.h:165-194) for bindings
 *     and harnesses: create / reset / prefill / decode / config /
 *     memory_stats / destroy.
 *
 * Status codes mirror the reference's exception types for the same
 * conditions: HIPLLM_INVALID_ARGUMENT = std::invalid_argument,
 * HIPLLM_OUT_OF_RANGE = std::out_of_range, HIPLLM_LENGTH_ERROR =
 * std::length_error, HIPLLM_RUNTIME_ERROR = std::runtime_error,
 * HIPLLM_OVERFLOW_ERROR = std::overflow_error. hipllm_last_error() returns the
 * message of the calling thread's last failure.
 *
 * GGML type ids: 0 F32, 1 F16, 6 Q5_0, 8 Q8_0, 12 Q4_K, 14 Q6_K
 * (metal_model.h:14-29). Quantized weights are passed in their native GGUF
 * row layout; `row_bytes` is the byte stride between rows.
 */
#ifndef HIPLLM_H
#define HIPLLM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    HIPLLM_OK = 0,
    HIPLLM_INVALID_ARGUMENT = 1,
    HIPLLM_OUT_OF_RANGE = 2,
    HIPLLM_LENGTH_ERROR = 3,
    HIPLLM_RUNTIME_ERROR = 4,
    HIPLLM_OVERFLOW_ERROR = 5,
};

const char* hipllm_last_error(void);
const char* hipllm_version(void);

/* ---------------------------------------------------------------- kernels */

/* Bit-exact FP32 dequantization of `rows` native rows of `k` values.
 * Replaces GgufDequantizer::row (model.cpp:543-578). */
int hipllm_dequant_rows(uint32_t type, const void* w, size_t row_bytes, size_t rows, size_t k, float* out,
                        void* stream);

/* Activation side-input of the GEMV: for every 16 values of x (k % 16 == 0)
 * one 64-byte group holding them as 24-bit fixed point in three signed-byte
 * digits (q = s2 * 65536 + s1 * 256 + s0, x ~= e q, |x - e q| <= e with
 * e = max|x| / 8355711 over the group), then the FP32 sum of the 16 values
 * and e: bytes s0[16] s1[16] s2[16], float sum, float e, 8 bytes padding.
 * xq holds k / 16 groups (4 k bytes, 16-byte aligned). The integer GEMV
 * multiplies quant bytes with the digits (v_dot4_i32_i8). Producers of GEMV
 * inputs (hipllm_rmsnorm, hipllm_attn_decode, hipllm_swiglu,
 * hipllm_gemv_swiglu, hipllm_gated_rmsnorm, hipllm_gate_mul) write this
 * form directly; hipllm_prep_x makes it from any x. */
int hipllm_prep_x(const float* x, void* xq, size_t k, void* stream);

/* Workspace bytes hipllm_gemv needs for an input of k values. */
size_t hipllm_gemv_workspace_bytes(size_t k);

/* Decode GEMV y[n] = W[n, k] x[k] (+ bias[n]); `workspace` holds
 * hipllm_gemv_workspace_bytes(k) bytes of device memory.
 * Replaces metal_gevm_{q5_0,q8_0,q4_k,q6_k,f32} via encode_vector_product
 * (metal_llm.metal:255-279, 708-781; metal_llm.mm:1891-1999) and CPULLM's
 * gevmt / gevmtb (cpu_llm.cpp:512-547). */
int hipllm_gemv(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* bias, float* y,
                size_t n, size_t k, void* workspace, void* stream);

/* hipllm_gemv without a workspace and without any allocation, for callers
 * that cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * The XGroup form of x goes to a static per-GPU device array of 256 KiB that
 * lives until the process ends, so k <= 65536 (HIPLLM_LENGTH_ERROR beyond).
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (other streams, other threads) race and must be ordered by the caller. The
 * stream must belong to the calling thread's current device. Same results
 * as hipllm_gemv, bit for bit. */
int hipllm_gemv_noalloc(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* bias, float* y,
                        size_t n, size_t k, void* stream);

/* GEMV with a caller-supplied XGroup input (hipllm_prep_x; quantized
 * weights read xq, F32 / F16 weights read x) and an optional residual:
 * y = W x (+ bias) (+ residual). `tiling` 0 picks the default; otherwise
 * 100 * R + OPR with R rows per 8-lane octet and OPR octets splitting each
 * row group's units: 108, 116, 132, 202, 204, 208, 216, 232, 401, 402, 404,
 * 408, 416, 432, 802, 804, 808, 816, 832. */
int hipllm_gemv_prepped(uint32_t type, const void* w, size_t row_bytes, const float* x, const void* xq,
                        const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                        void* stream);

/* The x16 tile-packed form of Q4_K and Q6_K weights (type 12 / 14), a
 * device-side layout of this backend (no counterpart in GGUF or the
 * reference): rows in tiles of 16 (a partial last tile zero-padded), one
 * tile-unit of 16 * 144 (Q4_K) or 16 * 210 (Q6_K) contiguous bytes per
 * 256-value super-block column: the 16 rows' blocks, byte for byte, ordered
 * the way the GEMV's lanes read them. hipllm_x16_bytes: its size for n rows
 * of k values (k % 256 == 0; 0 otherwise or for other types).
 * hipllm_pack_x16 writes it from native rows (packed 16-byte aligned; Q4_K
 * rows 16-byte, Q6_K rows 2-byte aligned). */
size_t hipllm_x16_bytes(uint32_t type, size_t n, size_t k);
int hipllm_pack_x16(uint32_t type, const void* w, size_t row_bytes, size_t n, size_t k, void* packed, void* stream);

/* An RMSNorm (cpu_llm.cpp:143-166) fused into an x16 GEMV; every field is
 * nullable and a null `norm` argument means none.
 * - Before the product (sumsq_in, eps; k <= 8192): xq holds the XGroup form
 *   of x * gamma for the raw row x, sumsq_in its k / 16 per-16-value sums of
 *   squares in double; the products are scaled by 1 / sqrt(mean + eps), so
 *   y = W (x * inv_rms * gamma) (+ bias) (+ residual), up to FP32 rounding.
 * - After the product (gamma_out, yq_out, sumsq_out; hipllm_gemv_x16 only,
 *   n % 16 == 0): y as usual, plus the XGroup form of y * gamma_out and the
 *   n / 16 double sums of squares of y: the input of a launch with a norm
 *   before its product.
 * Replaces the RMSNorm dispatches around the decode GEVMs
 * (metal_llm.mm:2776-2790, 2838-2848; metal_llm.metal:785-823). */
typedef struct HipllmX16Norm {
    const double* sumsq_in;
    float eps;
    const float* gamma_out;
    void* yq_out;
    double* sumsq_out;
} HipllmX16Norm;

/* Decode GEMV y = W x (+ bias) (+ residual) over x16-packed Q4_K or Q6_K
 * weights, with the integer products of the XGroup digits on the int8
 * matrix cores (v_mfma_i32_16x16x64_i8); xq as for hipllm_gemv_prepped.
 * Same arithmetic as the vector path (exact integer digit sums, FP32 scaling
 * per 16-group; Q6_K's three digit sums combined in FP32), results equal to
 * it within FP32 rounding.
 * `waves`: 0 picks the launch shape, else 1000 RT + 100 + W: W waves
 * per block (4, 8, 16) sharing RT 16-row tiles (1, 2), one unit in flight
 * per wave: 1104, 1108, 1116, 2104, 2108, 2116.
 * Replaces metal_gevm_q4_k_f32 / metal_gevm_q6_k_f32 via
 * encode_vector_product (metal_llm.metal:708-781; metal_llm.mm:1891-1999)
 * and gevmt for Q4_K / Q6_K rows (cpu_llm.cpp:512-547). */
int hipllm_gemv_x16(uint32_t type, const void* packed, const void* xq, const float* bias, const float* residual,
                    float* y, size_t n, size_t k, int waves, const HipllmX16Norm* norm, void* stream);

/* Two GEMVs of one RMSNorm-ed row over x16-packed weights (Q4_K or Q6_K
 * each) in one launch: y_a = W_a n and y_b = W_b n with n = rmsnorm(x) *
 * gamma (double sum of squares, every block normalising x itself; k <= 8192).
 * With conv_w, y_a is the input of a causal conv over its channels: y_a[c] =
 * silu(sum_j history[j][c] w[c][j] + (W_a n)[c] w[c][ksize - 1]) and the
 * (ksize - 1) x n_a history shifts by one row (ksize 2..4). With xq and
 * sumsq (both or neither) the norm comes from a producer's output norm data
 * instead (the XGroup form of x * gamma and its per-16-value double sums of
 * squares, as hipllm_gemv_x16 writes them); x and gamma are then unused. Replaces the
 * decode-step QKV / z GEVMs and the conv of encode_linear_attention
 * (moe_llm.mm:2436-2520; metal_llm.metal:708-781, 1320-1365). */
int hipllm_gemv_x16_pair(uint32_t type_a, const void* packed_a, size_t n_a, float* y_a, uint32_t type_b,
                         const void* packed_b, size_t n_b, float* y_b, size_t k, const float* x, const float* gamma,
                         float eps, const float* conv_w, float* history, size_t ksize, const void* xq,
                         const double* sumsq, void* stream);

/* The FFN gate/up pair over x16-packed weights of one type in one launch:
 * y = silu(Wg x) * (Wu x) (the sign-branched SiLU of cpu_llm.cpp:188-202),
 * and yq (nullable; n % 16 == 0) its XGroup form for the down projection.
 * Same launch shapes as hipllm_gemv_x16; `norm` as there (a norm before
 * the products only). Replaces the gate / up GEVMs and SwiGLU of
 * encode_decode_layer (metal_llm.mm:2850-2890; metal_llm.metal:708-781). */
int hipllm_gemv_x16_swiglu(uint32_t type, const void* gate, const void* up, const void* xq, float* y, void* yq,
                           size_t n, size_t k, int waves, const HipllmX16Norm* norm, void* stream);

/* One token's routed expert vectors over the x16 copy of a whole expert
 * block ([experts * n, k] rows packed as one matrix, n rows per expert,
 * n % 16 == 0): route j (j < routes <= 8) multiplies expert ids[j] (clamped
 * to experts - 1) or, when logits != nullptr, the route the kernel picks
 * itself (softmax / top-k / renormalisation of the token's router logits as
 * hipllm_router_topk computes them, experts <= 256; ids and weights stored
 * to ids_out / weights_out) by row j of xq (x_routed) or row 0 (rows ldx
 * values apart), into row j of y (ldy apart). packed2 != nullptr: the gate /
 * up pair, y = silu(Wg x) * (Wu x) and yq (nullable, ldy % 16 == 0) its
 * XGroup form. Launch shapes as hipllm_gemv_x16 (1104, 1108, 2104, 2108).
 * Replaces metal_expert_gemm_q4_k_f32 / metal_expert_gemm_q6_k_f32 and
 * metal_topk_f32 / metal_topk_renorm_f32 of encode_selected_moe
 * (metal_llm.metal:1424-1521; moe_llm.mm:2642-2790). */
int hipllm_gemv_x16_routed(uint32_t type, const void* packed, const void* packed2, const void* xq, size_t ldx,
                           int x_routed, float* y, void* yq, size_t ldy, size_t n, size_t k, size_t experts,
                           size_t routes, const int32_t* ids, const float* logits, int32_t* ids_out,
                           float* weights_out, int waves, void* stream);

/* One token's routed expert down projections, the shared expert's down
 * projection and the MoE combine in one launch, all on x16 copies: route j
 * (j < routes <= 8) multiplies expert ids[j]'s rows of the packed [experts *
 * n, k_r] down block (Q4_K or Q6_K) by XGroup row j of xq (ldx values
 * apart), the shared expert's packed [n, k_s] down matrix (Q4_K, Q6_K or
 * Q8_0, k_s <= 2048) multiplies the FP32 row sx, and y = residual + (sum_j
 * weights[j] down_j + sigmoid(sgate[0]) shared) (n % 16 == 0). norm_out
 * (nullable; gamma_out, yq_out and sumsq_out used) also writes the next
 * RMSNorm's data as hipllm_gemv_x16 with an output norm does. Replaces the
 * expert down GEMMs, shared-expert down GEVM and the weighted sum of
 * encode_selected_moe (moe_llm.mm:2790-2843; metal_llm.metal:1424-1521). */
/* Routed expert vectors of a prompt grouped by expert on x16 copies of the
 * whole expert block ([experts * n, k], n % 16 == 0, Q4_K or Q6_K): the
 * groups of hipllm_route_groups with vmax <= 4 (order, groups, ngroups;
 * max_groups = hipllm_route_groups_max(vectors, experts, vmax)); each group
 * reads its expert's tiles once for all its vectors. Vector v (an index
 * into the routed vectors) reads XGroup row v (x_routed) or v / routes of xq
 * (ldx values apart) and writes row v of y (ldy apart); packed2 != nullptr:
 * the gate / up pair, y = silu(Wg x) * (Wu x), yq (nullable) its XGroup
 * form. Replaces the expert GEMMs of encode_selected_moe for a prompt
 * (moe_llm.mm:2642-2843; metal_llm.metal:1424-1521). */
int hipllm_gemv_x16_grouped(uint32_t type, const void* packed, const void* packed2, const void* xq, size_t ldx,
                            int x_routed, size_t routes, float* y, void* yq, size_t ldy, size_t n, size_t k,
                            size_t experts, const int32_t* order, const int32_t* groups, const uint32_t* ngroups,
                            size_t max_groups, void* stream);

int hipllm_gemv_x16_moe_down(uint32_t type_r, const void* down_packed, const int32_t* ids, size_t experts,
                             const void* xq, size_t ldx, size_t k_r, uint32_t type_s, const void* shared_packed,
                             const float* sx, size_t k_s, const float* weights, const float* sgate,
                             const float* residual, float* y, size_t n, size_t routes,
                             const HipllmX16Norm* norm_out, void* stream);

/* hipllm_rmsnorm of the raw row x (gain gamma, k <= 8192, x and gamma
 * 16-byte aligned) followed by hipllm_gemv_prepped, in one launch: every
 * block normalises x into LDS (the same bits as hipllm_rmsnorm's XGroup
 * output) while its first weight loads are in flight. gamma nullptr: no norm,
 * the prologue makes hipllm_prep_x's XGroup form of x. Quantized types only;
 * `tiling` 0 picks the default, else 208, 216, 408 or 416. Replaces the
 * reference's RMSNorm + GEVM pair of each decode sub-block (encode_decode_layer,
 * metal_llm.mm:2758-2904; metal_llm.metal:785-823, 708-781). */
int hipllm_gemv_norm(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* gamma, float eps,
                     const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                     void* stream);

/* hipllm_rmsnorm followed by hipllm_gemv_swiglu in one launch, as
 * hipllm_gemv_norm; `tiling` 204 or 408 with yq, else also 208, 216, 416. */
int hipllm_gemv_swiglu_norm(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                            const float* gamma, float eps, float* y, void* yq, size_t n, size_t k, int tiling,
                            void* stream);

/* One GEMV of hipllm_gemv_multi_norm. mode 0: y = W x (+ bias) (+ residual),
 * quantized or F32 weights; mode 1: y = silu(W x) * (W2 x), quantized weights,
 * yq (nullable; n % 16 == 0) its XGroup form. reserved must be 0. */
typedef struct HipllmGemvJob {
    uint32_t type;
    uint32_t mode;
    const void* w;
    const void* w2;
    size_t row_bytes;
    const float* bias;
    const float* residual;
    float* y;
    void* yq;
    uint32_t n;
    uint32_t reserved;
} HipllmGemvJob;

/* Up to 3 GEMVs of one normalised row in one launch: every block normalises x
 * (k values, k % 32 == 0, k <= 8192; gain gamma) into LDS as
 * hipllm_rmsnorm does, then runs its job's rows (blocks of job p follow those
 * of job p - 1; tilings 208, 204 for mode 1 with yq, 108 for mode 1 without,
 * 132 for F32). norm and normq
 * (nullable, 16-byte aligned) receive the normalised row and its XGroup form.
 * For one decode row this replaces the RMSNorm and the projections that read
 * it (the DeltaNet QKV / z / alpha-beta GEVMs, moe_llm.mm:2436-2500; the
 * gated-attention Q / K / V GEVMs, 2238-2290; the router and shared-expert
 * gate/up of encode_routes and encode_selected_moe, 2642-2690, 2762-2790),
 * each a separate dispatch in the reference. */
int hipllm_gemv_multi_norm(const HipllmGemvJob* jobs, size_t count, const float* x, const float* gamma, float eps,
                           size_t k, float* norm, void* normq, void* stream);

/* Fused FFN gate/up GEMV + SwiGLU: y = silu(Wg x) * (Wu x); yq (nullable,
 * n % 16 == 0) receives the XGroup form of y. `tiling` 0 picks the default,
 * else one of the hipllm_gemv_prepped tilings; with yq only those whose
 * blocks hold whole 16-groups of y: 202, 204, 401, 402, 404, 408, 802, 804,
 * 808, 816. Replaces the gate/up
 * encode_vector_product pair + metal_swiglu_f32 (metal_llm.mm:2885-2894;
 * metal_llm.metal:895-911), cpu_llm.cpp:905-909. */
int hipllm_gemv_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                       const void* xq, float* y, void* yq, size_t n, size_t k, int tiling, void* stream);

/* The activation side-input of hipllm_gemm_mfma: per FP32 row
 * x[r * ldx + c] a power of two xscale[r] = 2^e, e chosen so the row's largest
 * magnitude over 2^e lies in [2^13, 2^14) (e = 0 for a zero or non-finite
 * row), and xh[r, c] (fp16, row-major, ld = k) = x / 2^e rounded to nearest
 * even. k % 8 == 0; x and xh 16-byte aligned. */
int hipllm_to_f16(const float* x, size_t ldx, void* xh, float* xscale, size_t m, size_t k, void* stream);

/* Prefill matmul Y[m, n] = X[m, k] W[n, k]^T (+ bias[n]) (+ residual[m, n])
 * with X given as scaled fp16 rows (hipllm_to_f16: xh, xscale), W in native
 * GGUF rows dequantized to fp16 (|w| < 65504), fp16 MFMA with FP32
 * accumulation; k % 128 == 0. `tile` < 0 picks the default, else
 * 0..3 = 128x32, 128x64, 256x64, 256x128 (weight rows x X rows per block),
 * 4, 5 = 128x128, 128x256 with each weight tile dequantized once into LDS
 * and shared by all four waves, 6 = 128x128 dequantized in registers.
 * `splits` 0 picks the default K split, else 1..1024 blocks along k: with
 * more than one, every split writes its partial sums to `workspace` (16-byte
 * aligned, hipllm_gemm_mfma_workspace_bytes) and a second launch adds them in
 * split order, then bias and residual, so results are the same on every
 * run; y may alias residual. Without enough workspace the default split
 * runs unsplit and an explicit one is rejected.
 * Replaces metal_gemm_{q5_0,q8_0,q4_k,q6_k,f32} via encode_matrix_product
 * (metal_llm.metal:196-250, 621-704; metal_llm.mm:1782-1889) and CPULLM's
 * gemmt / gemmtb (cpu_llm.cpp:591-607, 631-653). */
int hipllm_gemm_mfma(uint32_t type, const void* w, size_t row_bytes, const void* xh, const float* xscale,
                     const float* bias, const float* residual, float* y, size_t m, size_t n, size_t k, int tile,
                     int splits, void* workspace, size_t workspace_bytes, void* stream);
/* hipllm_rmsnorm of `rows` rows (cols contiguous values, cols % 16 == 0,
 * cols <= 8192; norm receives the normalised rows) and hipllm_to_f16 of its
 * output (xh, xscale) in one launch, with the same bits as the two.
 * Replaces the RMSNorm that precedes each prompt GEMM of cpu_prefill_layer
 * (cpu_llm.cpp:774-841). */
int hipllm_rmsnorm_f16(const float* x, const float* gamma, float* norm, void* xh, float* xscale, size_t rows,
                       size_t cols, float eps, void* stream);

/* The FFN gate / up matmuls of a prompt and their SwiGLU in three launches
 * instead of six: y[m, n] = silu(X Wg^T) * (X Wu^T) (the sign-branched SwiGLU
 * of cpu_llm.cpp:188-202) with X as for hipllm_gemm_mfma, Wg / Wu of one type
 * (Q4_K, Q6_K, Q8_0 or Q5_0) and the default tile and K split; both products'
 * partial planes go to `workspace` (16-byte aligned, at least
 * hipllm_gemm_swiglu_workspace_bytes(m, n, k) bytes) and one launch adds each
 * product's planes in split order and applies the SwiGLU: the same bits as
 * two hipllm_gemm_mfma calls and hipllm_swiglu. Replaces the gate / up GEMMs
 * and SwiGLU of cpu_prefill_layer (cpu_llm.cpp:774-841). */
size_t hipllm_gemm_swiglu_workspace_bytes(size_t m, size_t n, size_t k);
int hipllm_gemm_mfma_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const void* xh,
                            const float* xscale, float* y, size_t m, size_t n, size_t k, void* workspace,
                            size_t workspace_bytes, void* stream);

/* hipllm_gemm_mfma_swiglu with the SwiGLU rows written as the next matmul's
 * operand rows instead of FP32: yh / yscale as hipllm_to_f16 would make them
 * from y (the same bits; n % 8 == 0, n <= 32768, yh 16-byte aligned). The
 * down projection's input of cpu_prefill_layer (cpu_llm.cpp:774-841). */
int hipllm_gemm_mfma_swiglu_f16(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const void* xh,
                                const float* xscale, void* yh, float* yscale, size_t m, size_t n, size_t k,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes hipllm_gemm_mfma's K split takes for this shape, tile and
 * splits request (0: it runs unsplit). */
size_t hipllm_gemm_mfma_workspace_bytes(size_t m, size_t n, size_t k, int tile, int splits);

/* Workspace bytes hipllm_gemm needs for m rows of k values. */
size_t hipllm_gemm_workspace_bytes(size_t m, size_t k);

/* hipllm_gemm_mfma on FP32 X rows (ld = ldx), converted into `workspace`. */
int hipllm_gemm(uint32_t type, const void* w, size_t row_bytes, const float* x, size_t ldx, const float* bias,
                float* y, size_t m, size_t n, size_t k, void* workspace, void* stream);

/* Row RMSNorm y = x * (1/sqrt(mean(x^2) + eps) * gamma), double sum of
 * squares; yq (nullable) the XGroup form of y, rows of cols / 16 groups.
 * Replaces metal_rmsnorm_f32 (metal_llm.metal:785-823) and Vector::rmsnorm
 * (cpu_llm.cpp:143-166). */
int hipllm_rmsnorm(const float* x, const float* gamma, float* y, void* yq, size_t rows, size_t cols, float eps,
                   void* stream);

/* out[t, :] = dequant(table[ids[t]]); out-of-range ids give zeros.
 * Replaces metal_embedding_* (metal_llm.metal:1066-1162), embedding()
 * (cpu_llm.cpp:101-123). */
int hipllm_embed(uint32_t type, const void* table, size_t row_bytes, const int32_t* ids, size_t rows, size_t vocab,
                 size_t cols, float* out, void* stream);

/* NeoX RoPE on the Q and K heads of `rows` rows [Q | K | V] at positions
 * pos0 + r, with a cos/sin table (float2 per position and pair); rotated K
 * and V are written to the caches at those positions. Replaces
 * metal_rope_heads_f32 + metal_kv_cache_write_f32 (metal_llm.metal:928-990),
 * Vector::rope + cache append (cpu_llm.cpp:204-235, 874-886). */
int hipllm_rope_kv(float* qkv, const float* cos_sin, size_t rot, size_t hq, size_t hkv, size_t d, size_t pos0,
                   size_t rows, size_t row_stride, float* kcache, float* vcache, void* stream);

/* One decode token: hipllm_rope_kv on the raw [Q | K | V] row qkv at
 * position pos (the row itself is left unrotated) followed by
 * hipllm_attn_decode over [0, pos], in one launch pair: each attention block
 * rotates its query head, and the blocks holding the token's own key rotate
 * and write it (and V) to the caches first. Same bits as the two calls.
 * Replaces the same Metal and CPULLM steps as those two. */
int hipllm_attn_decode_rope(const float* qkv, const float* cos_sin, size_t rot, float* kcache, float* vcache,
                            float* out, void* outq, float* scratch, size_t hq, size_t hkv, size_t d, size_t pos,
                            float scale, void* stream);

/* hipllm_attn_decode_rope with the gated attention's output gate in the merge:
 * out = attention * sigmoid(gate) per element (gate: hq * d values), outq its
 * XGroup form. Replaces the decode attention and the sigmoid gate + multiply
 * of encode_full_attention (moe_llm.mm:2238-2434, the gate 2420-2428;
 * metal_llm.metal:1186-1197). */
int hipllm_attn_decode_rope_gated(const float* qkv, const float* cos_sin, size_t rot, float* kcache, float* vcache,
                                  const float* gate, float* out, void* outq, float* scratch, size_t hq, size_t hkv,
                                  size_t d, size_t pos, float scale, void* stream);

/* hipllm_split_qgate_norm and hipllm_attn_decode_rope_gated in one launch
 * (the same operations; caches bit for bit, outputs to within a few ulps of
 * the two launches'): mixed is the token's interleaved [Q_h | gate_h] row
 * (2 d per head), kv its [K | V] row; the Q and K heads are RMS-normalised
 * with q_gamma / k_gamma (eps), rotated, K / V written to the caches at pos,
 * and out = attention * sigmoid(gate_h), outq its XGroup form. Offered for
 * pos + 1 keys in 2 to 4 chunks of 64 (d 64 or 128; d 256 also) as one
 * block per head. Replaces the decode step of encode_full_attention
 * (moe_llm.mm:2238-2434; metal_llm.metal:1167-1197). */
int hipllm_attn_decode_qgate(const float* mixed, const float* kv, const float* q_gamma, const float* k_gamma,
                             float eps, const float* cos_sin, size_t rot, float* kcache, float* vcache, float* out,
                             void* outq, size_t hq, size_t hkv, size_t d, size_t pos, float scale, void* stream);

/* Scratch floats hipllm_attn_decode needs for up to max_len positions. */
size_t hipllm_attn_decode_scratch_floats(size_t hq, size_t d, size_t max_len);

/* One-token GQA attention over positions [0, len) of the caches; outq
 * (nullable) the XGroup form of out. Replaces metal_kv_cache_qk_f32 / metal_softmax_f32 /
 * metal_kv_cache_av_f32 (metal_llm.metal:826-890, 995-1061) and the decode
 * head loop (cpu_llm.cpp:893-906). */
int hipllm_attn_decode(const float* q, const float* kcache, const float* vcache, float* out, void* outq,
                       float* scratch, size_t hq, size_t hkv, size_t d, size_t len, float scale, void* stream);

/* Scratch bytes hipllm_argmax needs for n values. */
size_t hipllm_argmax_scratch_bytes(size_t n);

/* *out = index of the first maximum of x[0..n) (ties -> lower index).
 * Replaces metal_argmax_partial/finalize_f32 (metal_llm.metal:1544-1644),
 * greedy_token (cpu_llm.cpp:34-48). */
int hipllm_argmax(const float* x, size_t n, uint32_t* out, void* scratch, void* stream);

/* y = silu(g) * u (reference sign-branched sigmoid); yq (nullable) the
 * XGroup form of y. Replaces metal_swiglu_f32 (metal_llm.metal:895-911). */
int hipllm_swiglu(const float* g, const float* u, float* y, void* yq, size_t n, void* stream);

/* Causal prefill attention: query row r (position pos0 + r, heads at
 * q + r * q_stride) over cache positions [0, pos0 + r]. Replaces
 * metal_kv_cache_qk_f32 + softmax + av (metal_llm.metal:826-890, 995-1061)
 * and CPULLM's prefill head loop (cpu_llm.cpp:609-629, 316-329). */
int hipllm_attn_prefill(const float* q, size_t q_stride, const float* kcache, const float* vcache, float* out,
                        size_t out_stride, size_t rows, size_t hq, size_t hkv, size_t d, size_t pos0, float scale,
                        void* stream);

/* ----------------------------------------------------------- qwen35moe ops */

/* A batch of `vectors` GEMVs in one launch. Vector j: y[j * ldy, n) =
 * W_j x_j (+ bias) (+ residual[j]); with wu != NULL, y = silu(Wg_j x_j) *
 * (Wu_j x_j) and yq (nullable) gets its XGroup form (ld ldy / 16 groups).
 * With ids, W_j is expert ids[j] (byte offset ids[j] * expert_stride, ids
 * clamped to experts - 1) and x_j is row j (x_routed) or row j / routes of x
 * (ld ldx, xq ld ldx / 16 groups);
 * without ids every vector uses W and row j of x.
 * Replaces metal_expert_gemm_{q4_k,q6_k}_f32 (metal_llm.metal:1476-1521;
 * moe_llm.mm:2692-2760) and the per-row product of encode_product. */
int hipllm_gemv_batched(uint32_t type, const void* w, const void* wu, size_t row_bytes, const float* x,
                        const void* xq, const float* bias, const float* residual, float* y, void* yq, size_t n,
                        size_t k, size_t vectors, const int32_t* ids, size_t experts, size_t routes,
                        size_t expert_stride, int x_routed, size_t ldx, size_t ldy, void* stream);

/* Routed expert gate/up + SwiGLU with the routing in the same launch: every
 * block runs hipllm_router_topk's softmax / top-k / renormalisation on its
 * token's logits (experts <= 256, routes <= 8), then vector t * routes + q
 * computes y = silu(Wg_e x_t) * (Wu_e x_t) for expert e = ids_out[t, q] (yq:
 * nullable XGroup form, n % 16 == 0); ids_out and weights_out receive the
 * routes. Quantized weights, experts at expert_stride bytes. Replaces
 * metal_softmax_f32 / metal_topk_f32 / metal_topk_renorm_f32 and the expert
 * gate/up GEMMs with their SwiGLU (metal_llm.metal:826-890, 1424-1521;
 * moe_llm.mm:2642-2760). */
int hipllm_gemv_routed_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                              const void* xq, size_t ldx, float* y, void* yq, size_t n, size_t k, size_t tokens,
                              const float* logits, size_t ld_logits, size_t experts, size_t routes,
                              size_t expert_stride, int32_t* ids_out, float* weights_out, void* stream);

/* The shared expert's down projection with the MoE combine in its epilogue,
 * one token: y = residual + (sum_q weights[q] down[q n : (q + 1) n] +
 * sigmoid(sgate[0]) W x), the operations of hipllm_moe_combine (routes <= 8). x is raw FP32
 * (k <= 8192, 16-byte aligned; its XGroup form is made in the prologue);
 * quantized weights. Replaces the shared-expert down GEVM,
 * metal_expert_weighted_reduce_f32, the shared gate and the FFN residual
 * (metal_llm.metal:1525-1542, 1265-1276; moe_llm.mm:2790-2885). */
int hipllm_gemv_moe_combine(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* residual,
                            const float* down, const float* weights, const float* sgate, size_t routes, float* y,
                            size_t n, size_t k, void* stream);

/* y[m, n] = x[m, :k] . w[n, :k] in FP32 (row strides in floats): the router
 * logits of a prompt, reading each weight row once per 32 rows instead of once
 * per row. K is split over hipllm_matmul_f32_scratch_floats(m, n, k) floats of
 * scratch (partial sums added in split order, so results are deterministic;
 * with less scratch it runs unsplit). Replaces the router GEMM of
 * encode_routes for a prompt (moe_llm.mm:2642-2660). */
size_t hipllm_matmul_f32_scratch_floats(size_t m, size_t n, size_t k);
int hipllm_matmul_f32(const float* x, size_t ldx, const float* w, size_t ldw, float* y, size_t ldy, size_t m,
                      size_t n, size_t k, float* scratch, size_t scratch_floats, void* stream);

/* Routed vectors grouped by expert, for the expert products of several rows:
 * order = 0..n-1 sorted by ids (each clamped to experts - 1; in no fixed order
 * inside one expert); groups =
 * pairs {first index into order, expert | count << 16} of at most vmax vectors
 * of one expert; *ngroups = their count, at most
 * hipllm_route_groups_max(n, experts, vmax). n <= 16384, experts <= 1024. No
 * counterpart kernel in the reference, which runs one GEMM per route. */
size_t hipllm_route_groups_max(size_t n, size_t experts, size_t vmax);
int hipllm_route_groups(const int32_t* ids, size_t n, size_t experts, size_t vmax, int32_t* order, int32_t* groups,
                        uint32_t* ngroups, void* stream);

/* Routed expert products of several rows as the fp16 MFMA matmul
 * (hipllm_gemm_mfma's tile 1): one block row per group of
 * hipllm_route_groups (vmax <= 64), each reading its expert's weight tile
 * once for all of the group's vectors: y[j, :n] = W_e x_j for every routed
 * vector j, x_j = row j / routes of xh (hipllm_to_f16 rows and their
 * xscale, k values per row) or row j when x_routed; max_groups launch rows (those past *ngroups exit). Replaces the
 * per-route expert GEMMs of encode_selected_moe for a prompt
 * (moe_llm.mm:2692-2790; metal_llm.metal:1476-1521). */
int hipllm_gemm_gather(uint32_t type, const void* w, size_t row_bytes, const void* xh, const float* xscale, float* y,
                       size_t n, size_t k, size_t ldy, const int32_t* order, const int32_t* groups,
                       const uint32_t* ngroups, size_t max_groups, size_t expert_stride, size_t routes, int x_routed,
                       void* stream);

/* Per token: softmax over `experts` logits, top-k insertion (strict '>', the
 * lower id wins ties), renormalised weights. Replaces the router tail of
 * encode_routes (moe_llm.mm:2642-2690): metal_softmax_f32, metal_topk_f32,
 * metal_topk_renorm_f32 (metal_llm.metal:826-890, 1424-1474). */
int hipllm_router_topk(const float* logits, size_t ld, size_t tokens, size_t experts, size_t k, int32_t* ids,
                       float* weights, void* stream);

/* hipllm_moe_combine, then norm[t] = rmsnorm(out[t]) * gamma (normq, nullable:
 * its XGroup form), one block per token. Replaces the FFN residual of
 * encode_layer_experts and the next encode_rmsnorm (moe_llm.mm:2876-2883,
 * 2852-2855 of the next layer, 2954 after the last). */
int hipllm_moe_combine_norm(const float* residual, const float* down, const float* w, const float* shared,
                            const float* sgate, size_t ld_sgate, float* out, const float* gamma, float* norm,
                            void* normq, size_t tokens, size_t h, size_t k, float eps, void* stream);

/* out = residual + (sum_r w[t, r] down[t k + r] + sigmoid(sgate[t ld]) shared[t]).
 * Replaces metal_expert_weighted_reduce_f32 + shared-expert gate + residuals
 * (metal_llm.metal:1525-1542, 1265-1276; moe_llm.mm:2790-2885). */
int hipllm_moe_combine(const float* residual, const float* down, const float* w, const float* shared,
                       const float* sgate, size_t ld_sgate, float* out, size_t tokens, size_t h, size_t k,
                       void* stream);

/* decay = exp(softplus(alpha + dt_bias) a), beta = sigmoid(beta_raw).
 * Replaces the DeltaNet gate chain of encode_delta_net (moe_llm.mm:2462-2496;
 * metal_llm.metal:1186-1263). */
int hipllm_gdn_gates(const float* alpha, const float* beta_raw, size_t ld, const float* dt_bias, const float* a,
                     float* decay, float* beta, size_t tokens, size_t heads, void* stream);

/* Causal depthwise conv over [history; x] + SiLU, then history <- last k - 1
 * rows. Replaces metal_depthwise_conv1d_causal_f32, metal_conv_history_commit_f32
 * and the SiLU after them (metal_llm.metal:1320-1365, 1199-1211). */
int hipllm_conv1d_silu(const float* x, size_t ldx, float* history, const float* w, float* out, size_t ldo,
                       size_t tokens, size_t channels, size_t ksize, void* stream);

/* In place x <- x rsqrt(sum(x^2) + eps) per head vector. Replaces
 * metal_l2norm_heads_f32 (metal_llm.metal:1280-1316). */
int hipllm_l2norm_heads(float* x, size_t ld, size_t tokens, size_t heads, size_t d, float eps, void* stream);

/* Gated DeltaNet scan over `tokens` rows: per value head h (key head h % key
 * heads), S *= decay; delta = beta (v - S^T k); S += k delta^T;
 * o = S^T q / sqrt(d). State [value_heads, d, d] in place; d = 64 or 128.
 * Replaces metal_gdn_recurrence_f32 (metal_llm.metal:1370-1420). */
int hipllm_gdn_scan(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv, const float* decay,
                    const float* beta, float* state, float* out, size_t ldo, size_t tokens, size_t value_heads,
                    size_t key_heads, size_t d, void* stream);

/* hipllm_gdn_scan in the chunk-parallel form: 64-token chunks, each chunk's
 * delta-rule system (I + A) Delta = R solved through T = (I + A)^-1 for all
 * chunks at once, then one step per chunk carries the state (16 state
 * columns per block). Same arguments and results (to FP32 rounding) as
 * hipllm_gdn_scan; scratch holds hipllm_gdn_chunk_scratch_floats floats.
 * Replaces the serial scan of the prompt (metal_llm.metal:1370-1420) with the
 * chunked formulation the reference names as its next step
 * (QWEN36_35B_A3B_COMPATIBILITY.md:176-181, 476-479). */
size_t hipllm_gdn_chunk_scratch_floats(size_t tokens, size_t value_heads);
int hipllm_gdn_scan_chunked(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv,
                            const float* decay, const float* beta, float* state, float* out, size_t ldo,
                            size_t tokens, size_t value_heads, size_t key_heads, size_t d, float* scratch,
                            size_t scratch_floats, void* stream);

/* y = rmsnorm(o_head) gamma silu(z) per head (d <= 256); yq (nullable) the
 * XGroup form of y. Replaces the
 * state norm + SiLU(z) gate of encode_delta_net (moe_llm.mm:2614-2634). */
int hipllm_gated_rmsnorm(const float* o, size_t ldo, const float* gamma, const float* z, size_t ldz, float* y,
                         void* yq, size_t ldy, size_t tokens, size_t heads, size_t d, float eps, void* stream);

/* hipllm_conv1d_silu followed by hipllm_l2norm_heads on the first
 * norm_channels channels (the Q and K heads), in one pass: one block per
 * d-channel head segment (d = 64 or 128; channels and norm_channels
 * multiples of d). Replaces the same Metal kernels as those two. */
int hipllm_conv_l2norm(const float* x, size_t ldx, float* history, const float* w, float* out, size_t ldo,
                       size_t tokens, size_t channels, size_t ksize, size_t norm_channels, size_t d, float eps,
                       void* stream);

/* hipllm_gdn_gates + hipllm_gdn_scan + hipllm_gated_rmsnorm in one launch,
 * one block per value head: the gates come from the raw alpha / beta rows
 * (alpha[t * ld_ab + h], beta_raw[t * ld_ab + h]), the head's outputs are
 * normalised and gated by silu(z) in the block, y and its XGroup form yq
 * (nullable) are written. Replaces the same Metal kernels as those three. */
int hipllm_gdn_scan_gated(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv, const float* alpha,
                          const float* beta_raw, size_t ld_ab, const float* dt_bias, const float* a, float* state,
                          const float* z, size_t ldz, const float* gamma, float* y, void* yq, size_t ldy,
                          size_t tokens, size_t value_heads, size_t key_heads, size_t d, float eps, void* stream);

/* One decode token of a Gated DeltaNet layer after its projections (see
 * hipllm_gemv_x16_pair), one block per value head: qkv is the token's
 * convolved [Q (key_heads d) | K (key_heads d) | V (value_heads d)] row and
 * z its gate row; alpha and beta come from the F32 projection ab_w
 * ([alpha rows | beta rows], 2 value_heads x hidden, hidden <= 4096) of
 * rmsnorm(x) * x_gamma; then the Q / K head L2 norms and the step of
 * hipllm_gdn_scan_gated (gates, recurrence, gated RMSNorm; y and its XGroup
 * form yq, nullable). Replaces the decode-step use of the alpha / beta
 * GEVMs, L2 norms and recurrence of encode_linear_attention
 * (moe_llm.mm:2436-2640; metal_llm.metal:1320-1420). */
int hipllm_gdn_decode(const float* qkv, const float* x, const float* x_gamma, const float* ab_w, size_t hidden,
                      const float* dt_bias, const float* a, float* state, const float* z, const float* gamma, float* y,
                      void* yq, size_t value_heads, size_t key_heads, size_t d, float eps, void* stream);

/* Split the per-head interleaved [Q_h | gate_h] projection, RMSNorm Q and K
 * heads with their gammas, and lay out [Q | K | V] rows for RoPE + cache.
 * Replaces metal_split_interleaved_q_gate_f32 and the Q/K norms of
 * encode_full_attention (metal_llm.metal:1167-1184; moe_llm.mm:2258-2310). */
int hipllm_split_qgate_norm(const float* mixed, size_t ldm, const float* kv, size_t ldkv, const float* q_gamma,
                            const float* k_gamma, float* qkv, size_t ldqkv, float* gate, size_t ldg, size_t tokens,
                            size_t hq, size_t hkv, size_t d, float eps, void* stream);

/* y = a sigmoid(g); yq (nullable) the XGroup form of y. Replaces the
 * attention output gate of encode_full_attention (moe_llm.mm:2420-2428). */
int hipllm_gate_mul(const float* a, const float* g, float* y, void* yq, size_t n, void* stream);

/* ------------------------------------------------------------ handle API */

typedef struct HipllmModel HipllmModel;

typedef struct HipllmConfig {
    uint64_t layer_count;
    uint64_t embedding_size;
    uint64_t feed_forward_size;
    uint64_t attention_head_count;
    uint64_t kv_head_count;
    uint64_t head_size;
    uint64_t rotary_dimension;
    uint64_t vocabulary_size;
    uint64_t context_length;
    uint64_t parameter_count;
    uint64_t stored_weight_bytes;
    int32_t eos_token_id;
    float rope_theta;
    float norm_epsilon;
    char architecture[32];
    /* qwen35moe (zero for qwen2), metal_model.h:37-72 */
    uint64_t full_attention_interval;
    uint64_t expert_count;
    uint64_t expert_used_count;
    uint64_t expert_feed_forward_size;
    uint64_t shared_expert_feed_forward_size;
    uint64_t ssm_conv_kernel;
    uint64_t ssm_state_size;
    uint64_t ssm_group_count;
    uint64_t ssm_time_step_rank;
    uint64_t ssm_inner_size;
} HipllmConfig;

typedef struct HipllmMemoryStats {
    uint64_t weight_bytes;
    uint64_t kv_cache_bytes;
    uint64_t recurrent_state_bytes;
    uint64_t intermediate_bytes;
    int32_t intermediate_is_estimate;
} HipllmMemoryStats;

/* Parses a GGUF file with the streaming raw-tensor reader and derives the
 * model config, without touching a GPU. Replaces MetalRawModel's header
 * parsing + initialize_config (metal_model.cpp:451-688), as used by the
 * CLI's architecture probe (chat.cpp:1021-1024). */
int hipllm_inspect_gguf(const char* gguf_path, HipllmConfig* out);

/* Builds the backend the CLI's --gpu selection picks for the file
 * (chat.cpp:1019-1035): qwen35moe -> HipMoeLLM (MoeLLM, moe_llm.h:80-115),
 * otherwise HipLLM (MetalLLM(gguf_path, max_sequence), metal_llm.h:22-24).
 * device < 0 keeps the current HIP device; expert_cache_count is validated
 * like MoeLLM's (top-k <= n <= experts) and all experts stay resident. */
int hipllm_create(const char* gguf_path, size_t max_sequence, int device, HipllmModel** out);
int hipllm_create_ex(const char* gguf_path, size_t max_sequence, int device, size_t expert_cache_count,
                     HipllmModel** out);
void hipllm_destroy(HipllmModel* model);
int hipllm_reset(HipllmModel* model);
int hipllm_prefill(HipllmModel* model, const int32_t* ids, size_t count, int32_t* next_token);
int hipllm_decode(HipllmModel* model, int32_t id, int32_t* next_token);
int hipllm_config(const HipllmModel* model, HipllmConfig* out);
size_t hipllm_position(const HipllmModel* model);
size_t hipllm_max_sequence(const HipllmModel* model);
int hipllm_uses_gpu(const HipllmModel* model);
int hipllm_memory_stats(const HipllmModel* model, HipllmMemoryStats* out);
const char* hipllm_device_name(const HipllmModel* model);
/* MetalLLM::enable_profiling(csv_path, detailed_kernel_timestamps) /
 * disable_profiling (metal_llm.h:38-40): the reference's per-forward CSV
 * (profiler.cpp:619-632) and, with detailed != 0, its command / kernel /
 * operation sidecars (profiler.cpp:127-174). */
int hipllm_enable_profiling(HipllmModel* model, const char* csv_path, int detailed);
int hipllm_disable_profiling(HipllmModel* model);
/* The tokenizer tables of MetalModelConfig (metal_model.h:68-71), which
 * run_interactive and make_stop_tokens read (chat.cpp:708-726, 924-931):
 * entry i of tokenizer.ggml.tokens / tokenizer.ggml.merges (NULL past the
 * end) and tokenizer.ggml.pre ("" when absent). The strings live as long as
 * the model. */
size_t hipllm_vocabulary_count(const HipllmModel* model);
const char* hipllm_vocabulary_token(const HipllmModel* model, size_t index);
size_t hipllm_merge_count(const HipllmModel* model);
const char* hipllm_merge(const HipllmModel* model, size_t index);
const char* hipllm_tokenizer_pre(const HipllmModel* model);
/* Logits of the last prefill/decode (vocabulary_size floats, host memory). */
int hipllm_copy_logits(const HipllmModel* model, float* out, size_t count);
/* qwen2: 1 = batched (fp16 MFMA) prefill, 0 = token-serial prefill through
 * the FP32 decode kernels. qwen35moe: 1 = prompts of 16 or more rows run the
 * dense projections as fp16 MFMA matmuls (the router stays FP32), 0 = FP32
 * GEMVs for every row count. */
int hipllm_set_batched_prefill(HipllmModel* model, int enabled);

/* Decode path: 1 (default) = each decode step replays one recorded HIP graph
 * of the whole step (token and position read from device memory), 0 = its
 * kernels are launched one by one. Results agree to rounding (attention
 * splits follow the capacity rather than the length). Replaces the
 * reference's per-token command-buffer encoding (metal_llm.mm:3295-3385,
 * moe_llm.mm:3051-3141); no counterpart switch exists there. */
int hipllm_set_decode_graphs(HipllmModel* model, int enabled);
/* qwen2 only: 1 (default when the model has such projections) = the decode
 * GEMVs of Q4_K and Q6_K projections (fused QKV, attention output, FFN
 * gate / up and down, LM head) run on x16 tile-packed copies made at load
 * time (hipllm_gemv_x16; the copies count in memory_stats' weight_bytes),
 * 0 = on the GGUF rows.
 * HIPLLM_INVALID_ARGUMENT when the model has nothing to pack or is not
 * qwen2. No counterpart in the reference (a layout of this backend). */
int hipllm_set_packed_decode(HipllmModel* model, int enabled);
/* qwen2 only: 1 (default) = decode RMSNorms folded into the neighbouring
 * GEMVs where the model's forms allow (the GEMV prologue for rows of up to
 * 2048 values on GGUF rows; with x16 copies of every projection, the norm
 * data written by the attention output / FFN down GEMVs and applied by QKV,
 * gate / up and the LM head, HipllmX16Norm), 0 = every norm is its own
 * launch (hipllm_rmsnorm). Results agree to FP32 rounding. Replaces the
 * RMSNorm dispatches of encode_decode_layer (metal_llm.mm:2776-2848); no
 * counterpart switch exists there. */
int hipllm_set_fused_norms(HipllmModel* model, int enabled);
/* qwen35moe only: expert ids chosen for the last row of the last forward,
 * [layer_count, expert_used_count] (MoeLLM keeps them in RouteIds,
 * moe_llm.mm:2919-2925). */
int hipllm_copy_routes(const HipllmModel* model, int32_t* out, size_t count);
/* qwen35moe only, for parity checks of near-tie routes: with the probe on,
 * every forward keeps the last row's router logits (and shared-expert gate
 * logit) of each layer; hipllm_copy_router_logits reads them as
 * [layer_count, expert_count + 1] floats. Off by default. The reference
 * keeps them in its router scratch (encode_routes, moe_llm.mm:2642-2690). */
int hipllm_set_route_probe(HipllmModel* model, int enabled);
int hipllm_copy_router_logits(const HipllmModel* model, float* out, size_t count);
/* MoeLLM::expert_cache_count (moe_llm.h:104); 0 for qwen2 models. */
size_t hipllm_expert_cache_count(const HipllmModel* model);
/* MoeLLM::expert_cache_stats (moe_llm.h:105, ExpertCacheStats 12-20):
 * expert lookups since creation (tokens x routes x layers); every expert is
 * resident, so all are hits. Zero for qwen2 models. */
int hipllm_expert_cache_stats(const HipllmModel* model, uint64_t* hits, uint64_t* misses);

/* ------------------------------------------------------------ text front end */

/* Qwen byte-level BPE tokenizer: QwenTokenizer of chat.cpp:349-529 (qwen2 /
 * qwen35 pre-tokenizer, GPT-2 byte symbols, lowest-rank-first merges,
 * "<|...|>" special tokens matched longest first). Host code only: no GPU
 * call is made. Strings are NUL-terminated; a vocabulary or merge string
 * never holds a NUL byte in GPT-2 byte form. */
typedef struct HipllmTokenizer HipllmTokenizer;
int hipllm_tokenizer_create(const char* const* vocabulary, size_t vocabulary_count, const char* const* merges,
                            size_t merge_count, const char* tokenizer_pre, HipllmTokenizer** out);
/* From a loaded model's GGUF tables (run_interactive, chat.cpp:924-931). */
int hipllm_tokenizer_from_model(const HipllmModel* model, HipllmTokenizer** out);
void hipllm_tokenizer_destroy(HipllmTokenizer* tokenizer);
/* QwenTokenizer::encode (chat.cpp:379-399) of text[0, length). Writes up to
 * capacity ids and sets *count to the full number; HIPLLM_LENGTH_ERROR when
 * capacity is short (call again with *count). HIPLLM_RUNTIME_ERROR when the
 * vocabulary lacks a byte symbol the text needs (chat.cpp:509-518). */
int hipllm_tokenize(const HipllmTokenizer* tokenizer, const char* text, size_t length, int32_t* ids,
                    size_t capacity, size_t* count);
/* QwenTokenizer::id (chat.cpp:401-404): -1 when absent. */
int32_t hipllm_token_id(const HipllmTokenizer* tokenizer, const char* token);
/* QwenTokenizer::is_special (chat.cpp:423). */
int hipllm_token_is_special(const HipllmTokenizer* tokenizer, int32_t token);
/* QwenTokenizer::decode_piece (chat.cpp:406-421): the bytes of one token
 * ("" for special tokens and ids out of range), not NUL-terminated. Sets
 * *length; HIPLLM_LENGTH_ERROR when capacity is short. */
int hipllm_decode_piece(const HipllmTokenizer* tokenizer, int32_t token, char* out, size_t capacity,
                        size_t* length);
/* Byte ranges [begin, end) of the pre-tokenizer pieces of ordinary text
 * (pretokenize, chat.cpp:207-298), as 2 * *count values. */
int hipllm_pretokenize(const HipllmTokenizer* tokenizer, const char* text, size_t length, size_t* ranges,
                       size_t capacity, size_t* count);
/* ChatML prompt of one turn (chat_prompt, chat.cpp:655-659), same length
 * protocol as hipllm_decode_piece. */
int hipllm_chat_prompt(const char* system, const char* user, char* out, size_t capacity, size_t* length);
/* make_stop_tokens (chat.cpp:708-726): eos, <|im_end|>, </s>, then every
 * special token in id order, without repeats. */
int hipllm_stop_tokens(const HipllmModel* model, const HipllmTokenizer* tokenizer, int32_t* out, size_t capacity,
                       size_t* count);

/* GenerationStats (chat.h:20-41). */
typedef struct HipllmGenerationStats {
    double prefill_ms;
    double decode_ms;
    double total_ms;
    uint64_t prompt_tokens;
    uint64_t generated_tokens;
    uint64_t decode_steps;
    int32_t used_gpu;
    int32_t stopped;
    int32_t has_expert_cache_stats;
    uint64_t expert_cache_hits;
    uint64_t expert_cache_misses;
    HipllmMemoryStats memory;
} HipllmGenerationStats;
/* chat::run (chat.h:59-75, generate chat.cpp:831-878): reset, prefill, then
 * greedy emit/decode until a stop token or min(max_new_tokens,
 * max_sequence - count) tokens. sink (nullable) is called with each emitted
 * token; tokens (nullable) receives up to capacity of them and *generated
 * (nullable) their number; stats nullable. The errors of
 * validate_generation_request (chat.cpp:675-699) are HIPLLM_INVALID_ARGUMENT
 * / HIPLLM_RUNTIME_ERROR with the same messages. */
typedef void (*HipllmTokenSink)(int32_t token, void* user);
int hipllm_run(HipllmModel* model, const int32_t* ids, size_t count, size_t max_new_tokens, const int32_t* stop_ids,
               size_t stop_count, HipllmTokenSink sink, void* user, int32_t* tokens, size_t capacity,
               size_t* generated, HipllmGenerationStats* stats);
/* The "[chat] generation_stats ..." line (print_generation_stats,
 * chat.cpp:743-785), same length protocol as hipllm_decode_piece. */
int hipllm_format_generation_stats(const HipllmGenerationStats* stats, char* out, size_t capacity, size_t* length);
/* The chat command (run_cli, chat.cpp:998-1040) on stdin/stdout/stderr, with
 * the reference's options; --gpu is required (no CPU backend here). Returns
 * the exit status. */
int hipllm_chat_main(int argc, char** argv);

#ifdef __cplusplus
}
#endif

#endif /* HIPLLM_H */
