// Host-side launchers of the HipLLM kernels. Every launcher validates its
// arguments, launches on `stream` without allocating, and returns a status
// code from common.h (0 on success).
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

#include "common.h"

namespace hipllm {

int launch_dequant_rows(uint32_t type, const void* w, size_t row_bytes, size_t rows, size_t k, float* out,
                        hipStream_t stream);

// GEMV inputs travel as FP32 values x plus their XGroup form xq (k / 16
// groups, common.h); quantized weights read xq, F32 / F16 weights read x.
int launch_prep_x(const float* x, XGroup* xq, size_t k, hipStream_t stream);
int gemv_default_tiling(uint32_t n, uint32_t units, int mode, uint32_t vectors = 1, bool whole_groups = true);
int launch_gemv_prepped(uint32_t type, const void* w, size_t row_bytes, const float* x, const XGroup* xq,
                        const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                        hipStream_t stream);
int launch_gemv_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                       const XGroup* xq, float* y, XGroup* yq, size_t n, size_t k, int tiling, hipStream_t stream);

int launch_gemv_norm(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* gamma, float eps,
                     const float* bias, const float* residual, float* y, size_t n, size_t k, int tiling,
                     hipStream_t stream);
int launch_gemv_swiglu_norm(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                            const float* gamma, float eps, float* y, XGroup* yq, size_t n, size_t k, int tiling,
                            hipStream_t stream);
// One GEMV of a grouped launch (launch_gemv_multi_norm). mode 0: y = W x
// (+ bias) (+ residual); mode 1: y = silu(W x) * (W2 x) and, when yq is set,
// its XGroup form (n % 16 == 0). Quantized types and F32 (mode 0 only).
struct GemvJob {
    uint32_t type = 0;
    uint32_t mode = 0;
    const void* w = nullptr;
    const void* w2 = nullptr;
    size_t row_bytes = 0;
    const float* bias = nullptr;
    const float* residual = nullptr;
    float* y = nullptr;
    XGroup* yq = nullptr;
    uint32_t n = 0;
    uint32_t blocks = 0;  // set by the launcher
};
constexpr size_t kMultiJobs = 3;
// Up to kMultiJobs GEMVs of rmsnorm(x) * gamma (k values, k / 16 <= 512) in
// one launch, the norm in every block's prologue; norm / normq (nullable)
// receive the normalised row and its XGroup form.
int launch_gemv_multi_norm(const GemvJob* jobs, size_t count, const float* x, const float* gamma, float eps, size_t k,
                           float* norm, XGroup* normq, hipStream_t stream);
// y = residual + (sum_q weights[q] down[q n : (q + 1) n] + sigmoid(sgate[0]) W x)
// for one token: the shared expert's down projection with the MoE combine in
// its epilogue; x raw FP32 (XGroup form made in the prologue; quantized
// weights, k <= 8192).
int launch_gemv_moe_combine(uint32_t type, const void* w, size_t row_bytes, const float* x, const float* residual,
                            const float* down, const float* weights, const float* sgate, size_t routes, float* y,
                            size_t n, size_t k, hipStream_t stream);
// Expert gate/up + SwiGLU for tokens x routes vectors with the routes picked
// in the prologue from the router logits (softmax, top-k, renormalisation as
// launch_router_topk; experts <= 256, routes <= 8): vector t * routes + q
// multiplies row t of x by expert ids_out[t, q]; ids_out / weights_out
// receive the routes. Quantized weights.
int launch_gemv_routed_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const float* x,
                              const XGroup* xq, size_t ldx, float* y, XGroup* yq, size_t n, size_t k, size_t tokens,
                              const float* logits, size_t ld_logits, size_t experts, size_t routes,
                              size_t expert_stride, int32_t* ids_out, float* weights_out, hipStream_t stream);
// y[m, n] = x[m, :k] . w[n, :k] in FP32 (row strides ldx, ldw, ldy floats):
// the router logits of a prompt, each weight row read once per 32 rows. K
// split into matmul_f32_scratch_floats(m, n, k) floats of scratch (partial
// sums, added in split order; with less scratch it runs unsplit).
size_t matmul_f32_scratch_floats(size_t m, size_t n, size_t k);
int launch_matmul_f32(const float* x, size_t ldx, const float* w, size_t ldw, float* y, size_t ldy, size_t m, size_t n,
                      size_t k, float* scratch, size_t scratch_floats, hipStream_t stream);
// Routed vectors grouped by expert for the several-row expert products:
// order = 0..n-1 sorted by ids (each clamped to experts - 1; in no fixed
// order inside one expert); groups =
// pairs {first index into order, expert | count << 16}, at most vmax vectors
// of one expert each; *ngroups = the group count, at most
// route_groups_max(n, experts, vmax). n <= 16384, experts <= 1024.
size_t route_groups_max(size_t n, size_t experts, size_t vmax);
int launch_route_groups(const int32_t* ids, size_t n, size_t experts, size_t vmax, int32_t* order, int32_t* groups,
                        uint32_t* ngroups, hipStream_t stream);
// Expert products of several rows as the fp16 MFMA matmul, one block row per
// expert group (groups of at most kGatherRows vectors): y[j, :n] = W_e x_j
// for every routed vector j of the groups, x_j = row j / routes of xb (fp16,
// row scales xscale)
// or row j when x_routed; max_groups launch rows (those past *ngroups exit).
constexpr size_t kGatherRows = 64;
int launch_gemm_gather(uint32_t type, const void* w, size_t row_bytes, const void* xb, const float* xscale, float* y,
                       size_t n, size_t k, size_t ldy, const int32_t* order, const int32_t* groups,
                       const uint32_t* ngroups, size_t max_groups, size_t expert_stride, size_t routes, int x_routed,
                       hipStream_t stream);
int launch_gemv_batched(uint32_t type, const void* w, const void* wu, size_t row_bytes, const float* x,
                        const XGroup* xq, const float* bias, const float* residual, float* y, XGroup* yq, size_t n,
                        size_t k, size_t vectors, const int32_t* ids, size_t experts, size_t routes,
                        size_t expert_stride, int x_routed, size_t ldx, size_t ldy, hipStream_t stream);

// Q4_K / Q6_K rows in 16-row tiles, unit-major (the x16 packed form), and
// the decode GEMV over it on the int8 MFMA.
size_t x16_bytes(uint32_t type, size_t n, size_t k);
int launch_pack_x16(uint32_t type, const void* w, size_t row_bytes, size_t n, size_t k, void* packed,
                    hipStream_t stream);
// An RMSNorm fused into an x16 GEMV (all fields nullable): sumsq_in / eps for
// a norm before the product (xq then holds x * gamma), gamma_out / yq_out /
// sumsq_out for the data of a norm after y (plain GEMV only).
struct X16Norm {
    const double* sumsq_in;
    float eps;
    const float* gamma_out;
    XGroup* yq_out;
    double* sumsq_out;
    const float* x_in;      // the raw row normalised in every block (paired launch)
    const float* gamma_in;
};
int launch_gemv_x16(uint32_t type, const void* packed, const XGroup* xq, const float* bias, const float* residual,
                    float* y, size_t n, size_t k, int waves, hipStream_t stream, const X16Norm* norm = nullptr);
int launch_gemv_x16_swiglu(uint32_t type, const void* gate, const void* up, const XGroup* xq, float* y, XGroup* yq,
                           size_t n, size_t k, int waves, hipStream_t stream, const X16Norm* norm = nullptr);
// y_a = conv(W_a rmsnorm(x) * gamma) (conv + SiLU over history when conv_w
// is set, channel = row) and y_b = W_b rmsnorm(x) * gamma in one launch, each
// block normalising the raw row x itself (k <= 8192, x and gamma 16-byte
// aligned, ksize <= 4); or, with xq and sumsq (the producer's NORM 2 data:
// the XGroup form of x * gamma, per-16 sums of squares), from those (x and
// gamma unused).
int launch_gemv_x16_pair(uint32_t type_a, const void* packed_a, size_t n_a, float* y_a, uint32_t type_b,
                         const void* packed_b, size_t n_b, float* y_b, size_t k, const float* x, const float* gamma,
                         float eps, const float* conv_w, float* history, size_t ksize, hipStream_t stream,
                         const XGroup* xq = nullptr, const double* sumsq = nullptr);
// Routed expert vectors grouped by expert (launch_route_groups with vmax <=
// kX16GroupRows): each expert tile of the x16 copy of the whole [experts *
// n, k] block is read once per group and multiplied by every vector of it;
// vector index v reads input row v (x_routed) or v / routes and writes row
// v of y. packed2: the SwiGLU pair, yq (nullable) its XGroup form.
constexpr uint32_t kX16GroupRows = 4;
int launch_x16_grouped(uint32_t type, const void* packed, const void* packed2, const XGroup* xq, size_t ldx,
                       int x_routed, size_t routes, float* y, XGroup* yq, size_t ldy, size_t n, size_t k,
                       size_t experts, const int32_t* order, const int32_t* groups, const uint32_t* ngroups,
                       size_t max_groups, hipStream_t stream);
// One token's routed down projections (route j: expert ids[j]'s rows of the
// x16 copy of the whole [experts * n, k_r] down block times XGroup row j of
// xq), the shared expert's down projection (x16 copy, FP32 input sx of k_s
// <= 2048 values) and the MoE combine in one launch: y = residual + (sum_j
// weights[j] down_j + sigmoid(sgate[0]) shared); n % 16 == 0, routes <= 8.
// norm_out (nullable; gamma_out, yq_out, sumsq_out used): also the next
// RMSNorm's data, as a NORM 2 x16 launch writes it.
int launch_x16_moe_down(uint32_t type_r, const void* down_x16, const int32_t* ids, size_t experts, const XGroup* xq,
                        size_t ldx, size_t k_r, uint32_t type_s, const void* shared_x16, const float* sx, size_t k_s,
                        const float* weights, const float* sgate, const float* residual, float* y, size_t n,
                        size_t routes, hipStream_t stream, const X16Norm* norm_out = nullptr);
// One token's routed expert vectors over the x16 copy of a whole expert block
// ([experts * n, k], n rows per expert, n % 16 == 0): route j multiplies
// expert ids[j] (or, with logits, the router's top-k picked in the kernel,
// ids / weights stored to ids_out / weights_out) by row j of x (x_routed) or
// row 0, into row j of y (ldy apart). packed2 != nullptr: the gate / up
// SwiGLU pair (yq nullable: its XGroup form).
int launch_gemv_x16_routed(uint32_t type, const void* packed, const void* packed2, const XGroup* xq, size_t ldx,
                           int x_routed, float* y, XGroup* yq, size_t ldy, size_t n, size_t k, size_t experts,
                           size_t routes, const int32_t* ids, const float* logits, int32_t* ids_out,
                           float* weights_out, int waves, hipStream_t stream);

int gemm_default_tile(uint32_t m, uint32_t n, uint32_t k);
uint32_t gemm_default_splits(uint32_t m, uint32_t n, uint32_t k, int tile);
// X rows as fp16 MFMA operands with a power-of-two scale per row (xscale[m]).
int launch_to_f16(const float* x, size_t ldx, void* xh, float* xscale, size_t m, size_t k, hipStream_t stream);
// launch_rmsnorm (rows of k contiguous values, k % 16 == 0, k <= 8192) and
// launch_to_f16 of its output in one launch, with the same bits.
int launch_rmsnorm_f16(const float* x, const float* gamma, float* norm, void* xh, float* xscale, size_t m, size_t k,
                       float eps, hipStream_t stream);
// Bytes of the K-split partial planes launch_gemm_mfma uses for this shape
// (0 when it runs unsplit).
size_t gemm_split_bytes(size_t m, size_t n, size_t k, int tile, int splits);
// The FFN gate / up matmuls of a prompt (weights of one type, Q4_K / Q6_K /
// Q8_0 / Q5_0) and their SwiGLU: y = silu(X Wg^T) * (X Wu^T), the default
// tile and K split, both products' partial planes in ws (at least
// gemm_swiglu_bytes(m, n, k) bytes, 16-byte aligned) and one launch adding
// them in split order and applying the SwiGLU.
size_t gemm_swiglu_bytes(size_t m, size_t n, size_t k);
// With yh (and yscale) the SwiGLU rows go out as fp16 operand rows with their
// scales (to_f16's form; n % 8 == 0, n <= 32768) instead of FP32 y.
int launch_gemm_mfma_swiglu(uint32_t type, const void* wg, const void* wu, size_t row_bytes, const void* xb,
                            const float* xscale, float* y, size_t m, size_t n, size_t k, size_t ldy, void* ws,
                            size_t ws_bytes, hipStream_t stream, void* yh = nullptr, float* yscale = nullptr);
// With a K split the partial sums go to split_ws (gemm_split_bytes, 16-byte
// aligned) and are added in split order by a second launch; without enough
// workspace the default split runs unsplit and an explicit one is rejected.
int launch_gemm_mfma(uint32_t type, const void* w, size_t row_bytes, const void* xb, const float* xscale,
                     const float* bias, const float* residual, float* y, size_t m, size_t n, size_t k, int tile,
                     int splits, hipStream_t stream, size_t ldy = 0, void* split_ws = nullptr,
                     size_t split_ws_bytes = 0);
int launch_attn_prefill(const float* q, size_t q_stride, const float* kcache, const float* vcache, float* out,
                        size_t out_stride, size_t rows, size_t hq, size_t hkv, size_t d, size_t pos0, float scale,
                        hipStream_t stream);

int launch_rmsnorm(const float* x, const float* gamma, float* y, XGroup* yq, size_t rows, size_t cols, float eps,
                   hipStream_t stream);
int launch_embed(uint32_t type, const void* table, size_t row_bytes, const int32_t* ids, size_t rows, size_t vocab,
                 size_t cols, float* out, hipStream_t stream);
// dpos (optional, device): position of row 0 read on the device instead of
// pos0, so one recorded launch serves every decode step.
int launch_rope_kv(float* qkv, const float* cos_sin, size_t rot, size_t hq, size_t hkv, size_t d, size_t pos0,
                   size_t rows, size_t row_stride, float* kcache, float* vcache, hipStream_t stream,
                   const uint32_t* dpos = nullptr);
size_t attn_decode_scratch_floats(size_t hq, size_t d, size_t max_len);
// dpos (optional, device): len = *dpos + 1 read on the device; capacity then
// bounds it and fixes the launch shape.
int launch_attn_decode(const float* q, const float* kcache, const float* vcache, float* out, XGroup* outq,
                       float* scratch, size_t hq, size_t hkv, size_t d, size_t len, float scale, hipStream_t stream,
                       const uint32_t* dpos = nullptr, size_t capacity = 0);
// gate (nullable): out = attention * sigmoid(gate) per element (the gated
// attention's output gate), and outq its XGroup form.
int launch_attn_decode_rope(const float* qkv, const float* cos_sin, size_t rot, float* kcache, float* vcache,
                            float* out, XGroup* outq, float* scratch, size_t hq, size_t hkv, size_t d, size_t pos,
                            float scale, hipStream_t stream, const uint32_t* dpos = nullptr, size_t capacity = 0,
                            const float* gate = nullptr);
// Gated attention decode with its head norms in one launch (capacities of 2
// to 4 chunks, d 64 / 128 / 256; attn_decode_qgate_fits): mixed is the
// token's interleaved [Q_h | gate_h] row and kv its [K | V] row; Q and K
// heads are RMS-normalised with q_gamma / k_gamma (launch_split_qgate_norm's
// arithmetic) before the RoPE, then launch_attn_decode_rope with the gate.
bool attn_decode_qgate_fits(size_t max_len, size_t d);
int launch_attn_decode_qgate(const float* mixed, const float* kv, const float* q_gamma, const float* k_gamma,
                             float eps, const float* cos_sin, size_t rot, float* kcache, float* vcache, float* out,
                             XGroup* outq, size_t hq, size_t hkv, size_t d, size_t pos, float scale,
                             hipStream_t stream, const uint32_t* dpos = nullptr, size_t capacity = 0);
size_t argmax_scratch_bytes(size_t n);
int launch_argmax(const float* x, size_t n, uint32_t* out, void* scratch, hipStream_t stream);
int launch_swiglu(const float* g, const float* u, float* y, XGroup* yq, size_t n, hipStream_t stream);
int launch_add(const float* a, const float* b, float* y, size_t n, hipStream_t stream);

// qwen35moe operators (moe.hip).
int launch_router_topk(const float* logits, size_t ld, size_t tokens, size_t experts, size_t k, int32_t* ids,
                       float* weights, hipStream_t stream);
int launch_moe_combine(const float* residual, const float* down, const float* w, const float* shared,
                       const float* sgate, size_t ld_sgate, float* out, size_t tokens, size_t h, size_t k,
                       hipStream_t stream);
// launch_moe_combine, then norm = rmsnorm(out) * gamma (normq: nullable).
int launch_moe_combine_norm(const float* residual, const float* down, const float* w, const float* shared,
                            const float* sgate, size_t ld_sgate, float* out, const float* gamma, float* norm,
                            XGroup* normq, size_t tokens, size_t h, size_t k, float eps, hipStream_t stream);
int launch_gdn_gates(const float* alpha, const float* beta_raw, size_t ld, const float* dt_bias, const float* a,
                     float* decay, float* beta, size_t tokens, size_t heads, hipStream_t stream);
int launch_conv1d_silu(const float* x, size_t ldx, float* history, const float* w, float* out, size_t ldo,
                       size_t tokens, size_t channels, size_t ksize, hipStream_t stream);
int launch_l2norm_heads(float* x, size_t ld, size_t tokens, size_t heads, size_t d, float eps, hipStream_t stream);
int launch_gdn_scan(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv, const float* decay,
                    const float* beta, float* state, float* out, size_t ldo, size_t tokens, size_t value_heads,
                    size_t key_heads, size_t d, hipStream_t stream);
int launch_conv_l2norm(const float* x, size_t ldx, float* history, const float* w, float* out, size_t ldo,
                       size_t tokens, size_t channels, size_t ksize, size_t norm_channels, size_t d, float eps,
                       hipStream_t stream);
// The same recurrence as launch_gdn_scan in 64-token chunks (the chunk-
// parallel form; scratch: gdn_chunk_scratch_floats floats).
size_t gdn_chunk_scratch_floats(size_t tokens, size_t value_heads);
int launch_gdn_scan_chunked(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv,
                            const float* decay, const float* beta, float* state, float* out, size_t ldo,
                            size_t tokens, size_t value_heads, size_t key_heads, size_t d, float* scratch,
                            size_t scratch_floats, hipStream_t stream);
int launch_gdn_scan_gated(const float* q, const float* k, size_t ldqk, const float* v, size_t ldv, const float* alpha,
                          const float* beta_raw, size_t ld_ab, const float* dt_bias, const float* a, float* state,
                          const float* z, size_t ldz, const float* gamma, float* y, XGroup* yq, size_t ldy,
                          size_t tokens, size_t value_heads, size_t key_heads, size_t d, float eps,
                          hipStream_t stream);
// One decode token after the projections (launch_gemv_x16_pair made the
// convolved [Q | K | V] row qkv and the gate row z): alpha / beta from the
// F32 projection ab_w ([2 value_heads, hidden], hidden <= 4096) of
// rmsnorm(x) * x_gamma, the Q / K L2 norms, then launch_gdn_scan_gated's
// step; one block per value head.
int launch_gdn_decode(const float* qkv, const float* x, const float* x_gamma, const float* ab_w, size_t hidden,
                      const float* dt_bias, const float* a, float* state, const float* z, const float* gamma, float* y,
                      XGroup* yq, size_t value_heads, size_t key_heads, size_t d, float eps, hipStream_t stream);
int launch_gated_rmsnorm(const float* o, size_t ldo, const float* gamma, const float* z, size_t ldz, float* y,
                         XGroup* yq, size_t ldy, size_t tokens, size_t heads, size_t d, float eps,
                         hipStream_t stream);
int launch_split_qgate_norm(const float* mixed, size_t ldm, const float* kv, size_t ldkv, const float* q_gamma,
                            const float* k_gamma, float* qkv, size_t ldqkv, float* gate, size_t ldg, size_t tokens,
                            size_t hq, size_t hkv, size_t d, float eps, hipStream_t stream);
int launch_gate_mul(const float* a, const float* g, float* y, XGroup* yq, size_t n, hipStream_t stream);

}  // namespace hipllm
