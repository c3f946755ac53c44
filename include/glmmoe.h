/*
 * glmmoe.h -- C-ABI of the MI355X (gfx950) MoE-layer hot path for glmserve.
 *
 * Every pointer argument is a DEVICE pointer owned by the caller unless noted;
 * `stream` is a hipStream_t passed as void* (NULL = the null stream). No entry
 * point allocates device memory, frees or synchronizes; work is enqueued on
 * `stream`.
 * Return value: GLMMOE_OK (0) or a negative GLMMOE_ERR_* code; nothing throws
 * across this boundary (the reference's wrappers return void and print launch
 * errors, cuda/moe_expert.cu:126-129; callers here get a code instead).
 *
 * Data types: bf16 values travel as uint16_t bit patterns; fp32 as float.
 *
 * Citations are to the glmserve tree; each entry point names the
 * cuda/kernels.cuh launcher it replaces. include/glmmoe/kernels.hpp re-exposes
 * the reference-named subset as C++ inline functions.
 */
#ifndef GLMMOE_H
#define GLMMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GLMMOE_OK 0
#define GLMMOE_ERR_ARG (-1)       /* NULL pointer or non-positive size */
#define GLMMOE_ERR_SHAPE (-2)     /* shape outside what the kernels support */
#define GLMMOE_ERR_WORKSPACE (-3) /* workspace smaller than required */
#define GLMMOE_ERR_LAUNCH (-4)    /* the HIP runtime rejected a launch */

/* Library version string (host memory, static). */
const char* glmmoe_version(void);

/* ---- Router ---------------------------------------------------------------
 * Router-logit GEMM, logits[n,E] = x[n,H] . wr[E,H]^T, bf16 inputs, fp32 out.
 * Replaces gemm_linear(s.normed, d.router, ...) (src/model_gpu.cpp:1448 ->
 * gemm_fp32, cuda/kernels.cuh:37-38). Reduction order is fixed: K is cut into
 * chunks of 128, each chunk summed from zero in ascending K, chunk sums added
 * in ascending order -- restated by the CPU oracle, so logits are bit-exact.
 * xsum (nullable) receives sum_{k in chunk} x[t,k] as [n, H/128] fp32 (H %
 * 128 == 0), the activation group sums the W4A16 expert kernels consume.
 * workspace: device scratch of glmmoe_router_logits_workspace_bytes(n, H, E)
 * bytes (chunk partials of small batches; 0 bytes, NULL allowed, from 256
 * tokens with H % 128 == 0). Limits: H % 8 == 0, H <= 8192. */
size_t glmmoe_router_logits_workspace_bytes(int n, int H, int E);
int glmmoe_router_logits(const uint16_t* x, const uint16_t* wr, int n, int H, int E,
                         float* logits, float* xsum, void* workspace, size_t workspace_bytes,
                         void* stream);

/* Router logits from fp32 activations and fp32 router weights, with
 * gemm_fp32's argument list (cuda/kernels.cuh:37-38; the router call
 * gemm_linear(s.normed, d.router, nullptr, s.rlogits, n) of
 * src/model_gpu.cpp:1448): y[n, out] = bf16(x)[n, in] . bf16(W)[out, in]^T
 * (+ bias[out], nullable). x and W are rounded to bf16 (nearest-even) inside
 * the kernel; the sum is glmmoe_router_logits' fixed order, so y is
 * bit-identical to glmmoe_router_logits on the rounded inputs. No workspace.
 * Limits: in % 128 == 0, in <= 8192. */
int glmmoe_router_logits_f32(const float* x, const float* W, const float* bias, float* y,
                             int64_t n, int64_t in, int64_t out, void* stream);

/* Sigmoid top-k routing with score-correction bias.
 * Replaces moe_router (cuda/kernels.cuh:243-245, cuda/moe_router.cu:17-79):
 * same arguments and meaning. e_bias is nullable. Ties choose the lower
 * expert index; weights are the unbiased scores, normalized by their sum in
 * selection order when norm_topk != 0, then scaled by routed_scale.
 * Limits: 1 <= topk <= 8, topk <= E <= 512. */
int glmmoe_moe_router(const float* logits, const float* e_bias, int n, int E, int topk,
                      int norm_topk, float routed_scale, int* topk_ids, float* topk_weights,
                      void* stream);

/* Group the (token, slot) pairs by expert.
 * Replaces moe_dispatch (cuda/kernels.cuh:249-250, cuda/moe_dispatch.cu:16-45):
 * expert_offsets[E+1] (exclusive prefix), sorted_token_ids[n*topk],
 * sorted_row[n*topk] (the slot). Order within an expert is (token asc, slot
 * asc), deterministic, identical to the reference's serial counting sort.
 * Limits: E <= 512, n*topk <= 2^24. Ids outside [0,E) give GLMMOE_ERR_ARG
 * only if detected on the host side; on device they are skipped (counted in
 * no expert) -- callers pass router output, which is always in range. */
int glmmoe_moe_dispatch(const int* topk_ids, int n, int topk, int E, int* expert_offsets,
                        int* sorted_token_ids, int* sorted_row, void* stream);

/* ---- W4A16 weight format --------------------------------------------------
 * Reference format (src/tensor.cpp:53-63, cuda/kernels.cuh:259-268): per
 * matrix [rows, K] a packed u8 array [rows, K/2] (low nibble = even column,
 * value = nibble - 8) and scales [rows, K/group].
 * Native format ("packed"): 16-row x 128-K tiles of 1 KiB, tile (rb, kg) at
 * ((rb * K/128) + kg) * 1024 bytes; inside a tile lane l = r + 16*q (r = row
 * in block, q = 0..3) owns 16 bytes = K positions kg*128 + 32q + [0,32), one
 * dword per 8 positions, position 2s in nibble s and 2s+1 in nibble s+4.
 * Scales become bf16 [rows/16][K/128][16].
 * glmmoe_pack_w4a16 converts n_mats stacked reference matrices (experts) to
 * native. scales_dtype: 0 = fp32 (rounded to bf16, nearest-even), 1 = bf16.
 * Limits: rows % 16 == 0, K % 128 == 0, group_size == 128. */
size_t glmmoe_w4_packed_bytes(int rows, int K);       /* per matrix, weights */
size_t glmmoe_w4_packed_scale_bytes(int rows, int K); /* per matrix, scales */
int glmmoe_pack_w4a16(const uint8_t* qweight, const void* scales, int scales_dtype,
                      int n_mats, int rows, int K, int group_size, uint8_t* packed_q,
                      uint16_t* packed_scales, void* stream);

/* ---- Whole layer ------------------------------------------------------------
 * One GLM-5-class MoE layer: router GEMM -> routing -> dispatch -> grouped
 * W4A16 gate/up/SiLU -> grouped down -> deterministic combine with the shared
 * expert. Replaces the MoE branch of run_layer_step (src/model_gpu.cpp:
 * 1446-1495: gemm_linear(router), moe_router, cudaMemset, moe_expert_ffn_w4a16,
 * shared-expert gemm_w4a16 x3 + silu_mul + add_inplace). Output
 *   out[t] = sum_{s<topk, in slot order} w[t,s] * y_{e(t,s)}(x_t) + y_shared(x_t)
 * in fp32, the summation order of src/model_glm52.cpp:1133-1152.
 * All expert weights are in the native packed format; routed experts are
 * stacked (expert stride = packed bytes of one matrix). Shared expert
 * pointers may be NULL (no shared expert); when present its intermediate
 * size must equal moe_inter.
 * Limits: hidden % 256 == 0, moe_inter % 128 == 0, hidden <= 8192,
 * E <= 512, 1 <= topk <= 8. */
typedef struct glmmoe_w4a16_layer {
    int hidden;        /* H */
    int moe_inter;     /* I (per expert, also the shared expert's) */
    int n_experts;     /* E routed experts */
    int topk;
    int norm_topk;     /* norm_topk_prob */
    float routed_scale;/* routed_scaling_factor */
    const uint16_t* router_w;   /* [E, H] bf16 */
    const float* e_bias;        /* [E] fp32 or NULL */
    const uint8_t* gate_q;  const uint16_t* gate_s;  /* [E] x packed [I, H] */
    const uint8_t* up_q;    const uint16_t* up_s;    /* [E] x packed [I, H] */
    const uint8_t* down_q;  const uint16_t* down_s;  /* [E] x packed [H, I] */
    const uint8_t* sh_gate_q; const uint16_t* sh_gate_s; /* packed [I, H] or NULL */
    const uint8_t* sh_up_q;   const uint16_t* sh_up_s;
    const uint8_t* sh_down_q; const uint16_t* sh_down_s; /* packed [H, I] */
} glmmoe_w4a16_layer;

/* Device workspace carved by the layer call; every field points inside the
 * caller's workspace buffer. R = n*topk + n grouped rows (routed rows, then
 * one shared-expert row per token). */
typedef struct glmmoe_layer_ws {
    float* logits;        /* [n, E] */
    float* rpart;         /* router chunk partials (glmmoe_router_logits workspace) */
    float* xsum;          /* [n, H/128] */
    int* topk_ids;        /* [n, topk] */
    float* topk_w;        /* [n, topk] */
    int* expert_offsets;  /* [E + 2]: routed offsets, [E] = n*topk, [E+1] = R */
    int* sorted_token_ids;/* [R] */
    int* sorted_row;      /* [R] slot, -1 for shared rows */
    int* inv;             /* [n*topk]: grouped row of (t, s) */
    int* tiles;           /* [max_tiles * 4]: {expert, row0, nrows, j | m << 16} (tile j of
                             the expert's m full tiles, every batch size; 0 in the 4th
                             field for the 128-row layout's last tiles of 1-64 rows) */
    int* ntiles;          /* [3]: all tiles; the full tiles; the full and the 33-64-row
                             tiles. The 128-row layout (from 1024 grouped rows) lists the
                             full tiles (more than 64 rows, or every tile of the 16-row
                             layout), then each expert's last tile of 33-64 rows, then of
                             1-32 rows; the 16-row layout has only full tiles */
    uint16_t* h;          /* [R, I] SiLU(gate) * up: bf16 (16-row tiles) or fp16 scaled
                             by 2^e per row (128-row tiles; e in hsum, below) */
    float* hsum;          /* [R, I/128] group sums of h (decode kernels); from 1024 grouped rows
                             the int8 exponents of h's 32-feature blocks, [R, I/32] bytes */
    float* dpart;         /* [R, H] per-row expert outputs (unweighted): fp32 below 1024 grouped
                             rows (n*topk + n), bf16 (first half of the region) from there;
                             at least 256 * (H / 2048) * 16 KiB: before the down projection
                             it holds the gate/up kernel's split-item partials */
    unsigned int* sync;   /* [256] expert-kernel tickets (cleared by each call's router or dispatch kernel) */
    size_t bytes;         /* total workspace bytes */
} glmmoe_layer_ws;

size_t glmmoe_layer_workspace_bytes(const glmmoe_w4a16_layer* L, int n);
int glmmoe_layer_workspace_view(const glmmoe_w4a16_layer* L, int n, void* workspace,
                                glmmoe_layer_ws* view);

/* Runs the whole layer. x: [n, H] bf16; out: [n, H] fp32 (overwritten).
 * n == 0 returns GLMMOE_OK and touches nothing (x, out, workspace may be
 * NULL); so do the other layer, routing, dispatch (which then writes its
 * E + 1 zero offsets, as the reference's kernel does) and glmmoe_ref_* entry
 * points. */
int glmmoe_moe_layer_w4a16(const glmmoe_w4a16_layer* L, const uint16_t* x, int n,
                           float* out, void* workspace, size_t workspace_bytes,
                           void* stream);

/* The same layer on fp32 activations, the reference's s.normed as
 * run_layer_step hands it to the MoE branch (src/model_gpu.cpp:1446-1494):
 * x [n, H] fp32 is rounded to bf16 (nearest even) and the layer then runs
 * exactly as glmmoe_moe_layer_w4a16 on the rounded rows (bit-identical
 * output). Below 256 tokens the router kernel rounds the rows as it stages
 * them and writes the bf16 copy for the expert kernels (no extra launch);
 * from 256 tokens one conversion kernel runs first. The workspace is
 * glmmoe_layer_f32_workspace_bytes(L, n): the layer's plus the n x H bf16
 * copy at its end. */
size_t glmmoe_layer_f32_workspace_bytes(const glmmoe_w4a16_layer* L, int n);
int glmmoe_moe_layer_w4a16_f32(const glmmoe_w4a16_layer* L, const float* x, int n,
                               float* out, void* workspace, size_t workspace_bytes,
                               void* stream);

/* glmmoe_moe_layer_w4a16 with no workspace argument and no device allocation.
 * No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, serving loops that forbid hipMalloc). The
 * workspace is a device array of glmmoe_noalloc_scratch_bytes() (32 MiB) in
 * the library, one per GPU, kept until the process ends; a batch whose
 * glmmoe_layer_workspace_bytes exceeds it returns GLMMOE_ERR_WORKSPACE
 * (decode batches fit: 19 MiB at n = 64 on the GLM-5 layer). Every call on a
 * GPU uses that GPU's array: calls that overlap in time on one GPU (other
 * streams, other threads) race and must not be made. */
size_t glmmoe_noalloc_scratch_bytes(void);
int glmmoe_moe_layer_w4a16_noalloc(const glmmoe_w4a16_layer* L, const uint16_t* x, int n,
                                   float* out, void* stream);

/* The layer's routing alone: router logits and sigmoid top-k, as the layer
 * runs them (replaces gemm_linear on the router and moe_router,
 * src/model_gpu.cpp:1448-1450). topk_ids/topk_w: [n, topk], bit-identical to
 * moe_router on the fixed-order logits of glmmoe_router_logits. The workspace
 * is the layer's (its logits and xsum regions are written). */
int glmmoe_moe_route_w4a16(const glmmoe_w4a16_layer* L, const uint16_t* x, int n,
                           int* topk_ids, float* topk_w, void* workspace,
                           size_t workspace_bytes, void* stream);

/* The routed + shared expert stage alone, for callers that route elsewhere.
 * Replaces moe_expert_ffn_w4a16 (cuda/kernels.cuh:263-268) plus the shared
 * expert and add_inplace of src/model_gpu.cpp:1486-1494. topk_ids/topk_w are
 * [n, topk]; xsum may be NULL (then it is computed into the workspace). */
int glmmoe_expert_ffn_w4a16(const glmmoe_w4a16_layer* L, const uint16_t* x, int n,
                            const int* topk_ids, const float* topk_w, float* out,
                            void* workspace, size_t workspace_bytes, void* stream);

/* ---- FP8 (e4m3) experts ----------------------------------------------------
 * No counterpart in the reference's MoE (its FP8 code is the dense per-row-scale
 * GEMV gemm_fp8, cuda/kernels.cuh 55-57, cuda/fp8_gemm.cu 14-35, never called
 * by the forward; e4m3 decoding follows include/common.hpp 182-200). The same
 * layer semantics as glmmoe_moe_layer_w4a16 (GLM52Model::moe_mlp,
 * src/model_glm52.cpp 1096-1154) with:
 *   weights     e4m3 (OCP fn) [rows, K] plus fp32 scales per 128 x 128 block
 *               [rows/128, K/128]: w = e4m3(q) * scale. Codes 0x7f / 0xff are
 *               NaN on the MFMA (the reference host decoder reads them as
 *               +-480); quantizers must not emit them.
 *   activations x (bf16) quantized per token and 128 channels:
 *               scale = amax / 448 (1 for an all-zero group),
 *               q = e4m3(x / scale) rounded to nearest even, saturating at 448.
 *   h           SiLU(gate) * up quantized by the same rule before down.
 * The router still reads the bf16 x (glmmoe_router_logits). All expert GEMMs
 * run on 128-row tiles with fp8 MFMA. Shapes: H % 256 == 0, H <= 8192,
 * I % 128 == 0, E <= 512, topk <= 8. */

/* Bytes of one packed matrix [rows, K] (rows % 128 == 0, K % 128 == 0). */
size_t glmmoe_fp8_packed_bytes(int rows, int K);

/* Row-major e4m3 [n_mats, rows, K] -> the kernels' tile layout. Scales are
 * used as given ([n_mats, rows/128, K/128] fp32), no packing. */
int glmmoe_pack_fp8(const uint8_t* w, int n_mats, int rows, int K, uint8_t* packed,
                    void* stream);

/* x [n, K] bf16 -> q [n, K] e4m3 and scale [n, K/128] fp32 (K % 128 == 0), the
 * activation rule above. */
int glmmoe_quant_act_fp8(const uint16_t* x, int n, int K, uint8_t* q, float* scale,
                         void* stream);

typedef struct glmmoe_fp8_layer {
    int hidden;
    int moe_inter;
    int n_experts;
    int topk;
    int norm_topk;
    float routed_scale;
    const uint16_t* router_w;   /* [E, H] bf16 */
    const float* e_bias;        /* [E] fp32 or NULL */
    const uint8_t* gate_q;  const float* gate_s;  /* [E] x packed [I, H]; scales [E, I/128, H/128] */
    const uint8_t* up_q;    const float* up_s;    /* [E] x packed [I, H] */
    const uint8_t* down_q;  const float* down_s;  /* [E] x packed [H, I]; scales [E, H/128, I/128] */
    const uint8_t* sh_gate_q; const float* sh_gate_s; /* packed [I, H] or NULL */
    const uint8_t* sh_up_q;   const float* sh_up_s;
    const uint8_t* sh_down_q; const float* sh_down_s;
} glmmoe_fp8_layer;

typedef struct glmmoe_fp8_ws {
    float* logits;        /* [n, E] */
    float* rpart;         /* router chunk partials */
    uint8_t* xq;          /* [n, H] e4m3 */
    float* xscale;        /* [n, H/128] */
    int* topk_ids;        /* [n, topk] */
    float* topk_w;        /* [n, topk] */
    int* expert_offsets;  /* [E + 2] */
    int* sorted_token_ids;/* [R] */
    int* sorted_row;      /* [R] */
    int* inv;             /* [n*topk] */
    int* tiles;           /* [max_tiles * 4] */
    int* ntiles;          /* [1] */
    uint8_t* hq;          /* [R, I] e4m3 */
    float* hscale;        /* [R, I/128] */
    float* dpart;         /* [R, H] bf16 per-row expert outputs (fp32-sized region) */
    size_t bytes;
} glmmoe_fp8_ws;

size_t glmmoe_fp8_layer_workspace_bytes(const glmmoe_fp8_layer* L, int n);
int glmmoe_fp8_layer_workspace_view(const glmmoe_fp8_layer* L, int n, void* workspace,
                                    glmmoe_fp8_ws* view);
int glmmoe_moe_layer_fp8(const glmmoe_fp8_layer* L, const uint16_t* x, int n, float* out,
                         void* workspace, size_t workspace_bytes, void* stream);
int glmmoe_expert_ffn_fp8(const glmmoe_fp8_layer* L, const uint16_t* x, int n,
                          const int* topk_ids, const float* topk_w, float* out,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ---- Stage timing (diagnostics; no reference counterpart) -----------------
 * While enabled, every layer / expert-FFN call (W4A16 and FP8)
 * records a HIP event on its stream before and after each stage, in a ring of
 * GLMMOE_PROF_MAX_CALLS calls (events are created on the first enable; no
 * device memory is allocated). glmmoe_profile_read waits for the recorded
 * events and returns, per stage, the summed milliseconds and the number of
 * calls summed, then clears the ring. Stages: */
#define GLMMOE_STAGE_ROUTER_LOGITS 0
#define GLMMOE_STAGE_ROUTER_TOPK 1
#define GLMMOE_STAGE_DISPATCH 2
#define GLMMOE_STAGE_GATE_UP 3
#define GLMMOE_STAGE_DOWN 4
#define GLMMOE_STAGE_COMBINE 5
#define GLMMOE_N_STAGES 6
#define GLMMOE_PROF_MAX_CALLS 512
int glmmoe_profile_enable(int on);
int glmmoe_profile_read(float* stage_ms, int* n_calls);

/* ---- Reference-signature entry points ---------------------------------------
 * The cuda/kernels.cuh launchers that the MoE branch of the forward calls
 * (src/model_gpu.cpp:1448-1494), with the reference's arguments, weight
 * layouts and fp32 activations, for callers that keep the reference's call
 * sites; include/glmmoe/kernels.hpp exposes them under the reference's names
 * and argument lists. */

/* Routed W4A16 experts, replacing moe_expert_ffn_w4a16 (cuda/kernels.cuh:259-268,
 * cuda/moe_expert.cu:143-244) argument for argument: x fp32 [n, hidden];
 * gate/up qweight [E, moe_inter, hidden/2] u8 (low nibble = even column,
 * value nibble - 8) with fp32 scales [E, moe_inter, hidden/group_size]; down
 * [E, hidden, moe_inter/2] with [E, hidden, moe_inter/group_size]; out fp32
 * [n, hidden] overwritten with sum_s topk_weights[t,s] * y_{t,s} in slot
 * order (no shared expert, as in the reference).
 * The work runs the grouped kernels of glmmoe_expert_ffn_w4a16 on the native
 * packed copy of those weights (glmmoe_pack_w4a16, once at load time) that
 * glmmoe_ref_register_w4a16 associated with (gate_q, gate_sc, up_q, up_sc,
 * down_q, down_sc), in the
 * workspace glmmoe_ref_set_workspace registered for the current device, so
 * the call allocates nothing. x is rounded to bf16 (RNE) for those kernels and
 * the scales were rounded to bf16 when packed: results are within the W4A16
 * tolerance of the reference, not bit-identical. The scale arrays are not
 * read, only matched with the registration: weights updated in place, or
 * freed and reallocated, must be packed and registered again (registering
 * the same six pointers replaces the entry). Errors: GLMMOE_ERR_ARG when
 * these six pointers are not a registered set,
 * GLMMOE_ERR_WORKSPACE when no workspace of glmmoe_ref_workspace_bytes is
 * registered, GLMMOE_ERR_SHAPE for a shape other than the registered one.
 * Limits: group_size 128, hidden % 256 == 0, moe_inter % 128 == 0,
 * topk <= 8, E <= 512. The registry is a host-side table behind a lock;
 * registering or releasing while a call of the same weights is being
 * enqueued on another thread is the caller's race. */
int glmmoe_ref_register_w4a16(const uint8_t* gate_q, const float* gate_sc, const uint8_t* up_q,
                              const float* up_sc, const uint8_t* down_q, const float* down_sc,
                              const glmmoe_w4a16_layer* packed);
int glmmoe_ref_unregister_w4a16(const uint8_t* gate_q, const float* gate_sc, const uint8_t* up_q,
                                const float* up_sc, const uint8_t* down_q, const float* down_sc);
size_t glmmoe_ref_workspace_bytes(int n, int topk, int hidden, int moe_inter, int E);
int glmmoe_ref_set_workspace(void* workspace, size_t bytes);
int glmmoe_ref_moe_expert_ffn_w4a16(const float* x, const int* topk_ids, const float* topk_weights,
                                    const uint8_t* gate_q, const float* gate_sc,
                                    const uint8_t* up_q, const float* up_sc,
                                    const uint8_t* down_q, const float* down_sc, int n, int topk,
                                    int hidden, int moe_inter, int E, int group_size, float* out,
                                    void* stream);

/* Routed experts with fp32 weights, replacing moe_expert_ffn (cuda/kernels.cuh:
 * 252-257, cuda/moe_expert.cu:32-130): gate/up [E, moe_inter, hidden], down
 * [E, hidden, moe_inter] fp32; out [n, hidden] overwritten with
 * sum_s w[t,s] * down_e(silu(gate_e x) * up_e x) in slot order. One workgroup
 * per token, fp32 throughout (the reference's per-token structure; fp32
 * experts are not a served format). Limit: topk * moe_inter <= 40960. */
int glmmoe_ref_moe_expert_ffn(const float* x, const int* topk_ids, const float* topk_weights,
                              const float* gate_w, const float* up_w, const float* down_w, int n,
                              int topk, int hidden, int moe_inter, int E, float* out,
                              void* stream);

/* y[n, out] = x[n, in] . W[out, in]^T (+ bias), fp32 in and out, replacing
 * gemm_w4a16 (cuda/kernels.cuh:50-52, cuda/int4_gemm.cu:15-48): qW [out,
 * ceil(in/2)] u8, scales [out, ceil(in/group_size)] fp32, bias nullable; the
 * shared expert's linears. Any shape; in % 8 == 0 with group_size % 8 == 0
 * takes the staged path (a workgroup per 16 rows, tokens in blocks of 8). */
int glmmoe_ref_gemm_w4a16(const float* x, const uint8_t* qW, const float* scales,
                          const float* bias, float* y, int64_t n, int64_t in, int64_t out,
                          int64_t group_size, void* stream);

/* The same product with e4m3 weights [out, in] and an optional fp32 scale per
 * row, replacing gemm_fp8 (cuda/kernels.cuh:55-57, cuda/fp8_gemm.cu:14-44).
 * e4m3 is the OCP "fn" encoding: codes 0x7f / 0xff decode to NaN (as the
 * reference's device conversion does). */
int glmmoe_ref_gemm_fp8(const float* x, const uint8_t* fp8W, const float* w_scale,
                        const float* bias, float* y, int64_t n, int64_t in, int64_t out,
                        void* stream);

/* out = silu(g) * u and y += x over n floats, replacing silu_mul and
 * add_inplace (cuda/kernels.cuh:281-282, cuda/mla_glue.cu:10-28). */
int glmmoe_ref_silu_mul(const float* g, const float* u, float* out, int64_t n, void* stream);
int glmmoe_ref_add_inplace(float* y, const float* x, int64_t n, void* stream);

/* GGUF block-quantized weights (the ggml block formats of src/gguf_quant.cpp:
 * qtype 0 F32, 1 F16, 8 Q8_0, 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K, 18 IQ3_XXS,
 * 23 IQ4_XS), dequantized inside the kernels bit-identically to the
 * reference's CPU dequantizer; products and sums in fp32.
 * glmmoe_ref_gemm_q replaces gemm_q (cuda/kernels.cuh:63-66): y[n,out] =
 * x[n,in] . W^T (+ bias), row o of W at qW + o * row_bytes.
 * glmmoe_ref_moe_expert_ffn_q replaces moe_expert_ffn_q (cuda/kernels.cuh:
 * 117-123, cuda/qgemm.cu:1505-1639) argument for argument: gate/up rows
 * [E, moe_inter, hidden], down [E, hidden, moe_inter], row o of expert e at
 * base + (e * out + o) * row_bytes; h_act [n, topk, moe_inter] and dpart
 * [n * topk, hidden] are caller scratch; out [n, hidden] is overwritten with
 * sum_s topk_w[t,s] * y_{t,s} in slot order. With `dispatch` (int scratch of
 * 3E + 1 + n*topk, nullable) the routed rows are grouped by expert first so
 * each weight row is read once per 8 rows of its expert; without it every
 * routed row reads its expert's rows (the reference's token-major path).
 * gu_part (the reference's split-K partials) is accepted and not used.
 * Limits: every row length a multiple of its type's block and of 8,
 * row_bytes at least the blocks of a row, E <= 4096. */
int glmmoe_ref_gemm_q(uint32_t qtype, const float* x, const uint8_t* qW, const float* bias,
                      float* y, int64_t n, int64_t in, int64_t out, int64_t row_bytes,
                      void* stream);
int glmmoe_ref_moe_expert_ffn_q(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                                const float* x, const int* topk_ids, const float* topk_w,
                                const uint8_t* gate_q, const uint8_t* up_q, const uint8_t* down_q,
                                int n, int topk, int hidden, int moe_inter, int E,
                                int64_t gate_row_bytes, int64_t up_row_bytes,
                                int64_t down_row_bytes, float* h_act, float* dpart, float* out,
                                int* dispatch, float* gu_part, void* stream);

/* int8-activation twins (cuda/kernels.cuh:68-83, 124-135; cuda/qgemm.cu:
 * 104-303, 556-587, 775-779, 1656-1670).
 * glmmoe_ref_qtype_has_i8 replaces qtype_has_i8: 1 for Q8_0, Q3_K, Q4_K,
 * Q5_K, Q6_K, IQ3_XXS and IQ4_XS, 0 otherwise.
 * glmmoe_ref_quantize_act_q8 replaces quantize_act_q8: xq [n, in] int8 and
 * xs [n, in/32] fp32 with, per 32-element block, xs = absmax / 127 and
 * xq = round-half-even(x * (1 / xs)) (0 for an all-zero block); in % 32 == 0.
 * glmmoe_ref_gemm_q_i8 replaces gemm_q_i8: gemm_q with pre-quantized
 * activations; each 8-weight fragment is an int8 dot,
 * y += xs * (ds * dot(wq, xq) - dm * sum(xq)).
 * glmmoe_ref_moe_expert_ffn_q_i8 replaces moe_expert_ffn_q_i8 argument for
 * argument: moe_expert_ffn_q with x as (xq, xs); h_act (fp32) is quantized
 * into hq [n*topk, moe_inter] and hs [n*topk, moe_inter/32] between the
 * gate/up and down phases.
 * Limits: as gemm_q / moe_expert_ffn_q, every type int8-capable, in / hidden /
 * moe_inter multiples of 32, xq and hq 4-byte aligned (else GLMMOE_ERR_SHAPE). */
int glmmoe_ref_qtype_has_i8(uint32_t qtype);
int glmmoe_ref_quantize_act_q8(const float* x, int64_t n, int64_t in, int8_t* xq, float* xs,
                               void* stream);
int glmmoe_ref_gemm_q_i8(uint32_t qtype, const int8_t* xq, const float* xs, const uint8_t* qW,
                         const float* bias, float* y, int64_t n, int64_t in, int64_t out,
                         int64_t row_bytes, void* stream);
int glmmoe_ref_moe_expert_ffn_q_i8(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                                   const int8_t* xq, const float* xs, const int* topk_ids,
                                   const float* topk_w, const uint8_t* gate_q,
                                   const uint8_t* up_q, const uint8_t* down_q, int n, int topk,
                                   int hidden, int moe_inter, int E, int64_t gate_row_bytes,
                                   int64_t up_row_bytes, int64_t down_row_bytes, float* h_act,
                                   int8_t* hq, float* hs, float* dpart, float* out, int* dispatch,
                                   float* gu_part, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* GLMMOE_H */
