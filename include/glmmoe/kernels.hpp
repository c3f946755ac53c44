// glmmoe/kernels.hpp -- C++ face of the MI355X MoE-layer library with the
// names and argument lists of glmserve's launch API (cuda/kernels.cuh:241-268)
// for the MoE hot path.
//
// A caller written against kernels.cuh switches by including this header in
// place of kernels.cuh for the MoE calls and passing hipStream_t streams
// (any pointer converts to the void* stream parameter). Differences from the
// reference, by design:
//   * functions return the C-ABI status (int, 0 = ok) instead of void; a call
//     site that ignores the result compiles unchanged;
//   * the router logits come from glmmoe_router_logits (bf16 in, fixed
//     reduction order) rather than gemm_fp32 on fp32 activations;
//   * expert weights live in the native packed W4A16 layout produced once at
//     load time by pack_w4a16 (from the reference's qweight/scales layout). The
//     fast form of the routed + shared expert stage is one call
//     (moe_expert_ffn_w4a16 with a glmmoe_w4a16_layer) instead of
//     moe_expert_ffn_w4a16 + 3 gemm_w4a16 + silu_mul + add_inplace; those
//     launchers also exist with the reference's argument lists (below), the
//     W4A16 experts after a one-time registration of the packed copy.
// Define GLMMOE_GLMSERVE_NAMESPACE to also make these visible as
// glmserve::cuda::* (only when kernels.cuh is not included in the same unit).
#pragma once

#include <cstddef>
#include <cstdint>

#include "../glmmoe.h"

namespace glmmoe {
namespace compat {

// cuda/kernels.cuh:243-245
inline int moe_router(const float* logits, const float* e_bias, int n, int E, int topk,
                      bool norm_topk, float routed_scale, int* topk_ids, float* topk_weights,
                      void* s = nullptr) {
    return glmmoe_moe_router(logits, e_bias, n, E, topk, norm_topk ? 1 : 0, routed_scale,
                             topk_ids, topk_weights, s);
}

// cuda/kernels.cuh:249-250
inline int moe_dispatch(const int* topk_ids, int n, int topk, int E, int* expert_offsets,
                        int* sorted_token_ids, int* sorted_row, void* s = nullptr) {
    return glmmoe_moe_dispatch(topk_ids, n, topk, E, expert_offsets, sorted_token_ids,
                               sorted_row, s);
}

// Router-logit GEMM (replaces gemm_linear(s.normed, d.router, ...) at
// src/model_gpu.cpp:1448 for bf16 activations and router weights).
inline int router_logits(const uint16_t* x_bf16, const uint16_t* wr_bf16, int n, int H, int E,
                         float* logits, float* xsum, void* workspace, size_t workspace_bytes,
                         void* s = nullptr) {
    return glmmoe_router_logits(x_bf16, wr_bf16, n, H, E, logits, xsum, workspace,
                                workspace_bytes, s);
}

// Load-time repack of reference-layout W4 experts (src/model_gpu.cpp:913-1010
// uploads qweight [E, rows, K/2] and scales [E, rows, K/g]).
inline int pack_w4a16(const uint8_t* qweight, const float* scales_f32, int n_mats, int rows,
                      int K, int group_size, uint8_t* packed_q, uint16_t* packed_scales,
                      void* s = nullptr) {
    return glmmoe_pack_w4a16(qweight, scales_f32, 0, n_mats, rows, K, group_size, packed_q,
                             packed_scales, s);
}
inline int pack_w4a16_bf16_scales(const uint8_t* qweight, const uint16_t* scales_bf16, int n_mats,
                                  int rows, int K, int group_size, uint8_t* packed_q,
                                  uint16_t* packed_scales, void* s = nullptr) {
    return glmmoe_pack_w4a16(qweight, scales_bf16, 1, n_mats, rows, K, group_size, packed_q,
                             packed_scales, s);
}

// Routed + shared experts with caller routing (cuda/kernels.cuh:263-268 plus
// the shared-expert chain of src/model_gpu.cpp:1486-1494); out is overwritten.
inline int moe_expert_ffn_w4a16(const glmmoe_w4a16_layer& layer, const uint16_t* x_bf16, int n,
                                const int* topk_ids, const float* topk_weights, float* out,
                                void* workspace, size_t workspace_bytes, void* s = nullptr) {
    return glmmoe_expert_ffn_w4a16(&layer, x_bf16, n, topk_ids, topk_weights, out, workspace,
                                   workspace_bytes, s);
}

// The whole MoE branch of run_layer_step (src/model_gpu.cpp:1446-1495).
inline int moe_layer_w4a16(const glmmoe_w4a16_layer& layer, const uint16_t* x_bf16, int n,
                           float* out, void* workspace, size_t workspace_bytes,
                           void* s = nullptr) {
    return glmmoe_moe_layer_w4a16(&layer, x_bf16, n, out, workspace, workspace_bytes, s);
}

inline size_t moe_layer_workspace_bytes(const glmmoe_w4a16_layer& layer, int n) {
    return glmmoe_layer_workspace_bytes(&layer, n);
}

// The same branch on run_layer_step's fp32 s.normed, passed unchanged
// (src/model_gpu.cpp:1446-1494); workspace of moe_layer_f32_workspace_bytes.
inline int moe_layer_w4a16(const glmmoe_w4a16_layer& layer, const float* x_f32, int n, float* out,
                           void* workspace, size_t workspace_bytes, void* s = nullptr) {
    return glmmoe_moe_layer_w4a16_f32(&layer, x_f32, n, out, workspace, workspace_bytes, s);
}

inline size_t moe_layer_f32_workspace_bytes(const glmmoe_w4a16_layer& layer, int n) {
    return glmmoe_layer_f32_workspace_bytes(&layer, n);
}

// ---- The reference's own argument lists (fp32 activations, reference weight
// layouts). moe_expert_ffn_w4a16 needs the weights registered once at load
// time (glmmoe_ref_register_w4a16 with their packed copy) and a workspace
// registered per device (glmmoe_ref_set_workspace); the rest need nothing.

// cuda/kernels.cuh:263-268
inline int moe_expert_ffn_w4a16(const float* x, const int* topk_ids, const float* topk_weights,
                                const uint8_t* gate_q, const float* gate_sc, const uint8_t* up_q,
                                const float* up_sc, const uint8_t* down_q, const float* down_sc,
                                int n, int topk, int hidden, int moe_inter, int E, int group_size,
                                float* out, void* s = nullptr) {
    return glmmoe_ref_moe_expert_ffn_w4a16(x, topk_ids, topk_weights, gate_q, gate_sc, up_q,
                                           up_sc, down_q, down_sc, n, topk, hidden, moe_inter, E,
                                           group_size, out, s);
}

// cuda/kernels.cuh:254-257
inline int moe_expert_ffn(const float* x, const int* topk_ids, const float* topk_weights,
                          const float* gate_w, const float* up_w, const float* down_w, int n,
                          int topk, int hidden, int moe_inter, int E, float* out,
                          void* s = nullptr) {
    return glmmoe_ref_moe_expert_ffn(x, topk_ids, topk_weights, gate_w, up_w, down_w, n, topk,
                                     hidden, moe_inter, E, out, s);
}

// cuda/kernels.cuh:50-52
inline int gemm_w4a16(const float* x, const uint8_t* qW, const float* scales, const float* bias,
                      float* y, int64_t n, int64_t in, int64_t out, int64_t group_size,
                      void* s = nullptr) {
    return glmmoe_ref_gemm_w4a16(x, qW, scales, bias, y, n, in, out, group_size, s);
}

// cuda/kernels.cuh:55-57
inline int gemm_fp8(const float* x, const uint8_t* fp8W, const float* w_scale, const float* bias,
                    float* y, int64_t n, int64_t in, int64_t out, void* s = nullptr) {
    return glmmoe_ref_gemm_fp8(x, fp8W, w_scale, bias, y, n, in, out, s);
}

// cuda/kernels.cuh:281-282
inline int add_inplace(float* y, const float* x, int64_t n, void* s = nullptr) {
    return glmmoe_ref_add_inplace(y, x, n, s);
}
inline int silu_mul(const float* g, const float* u, float* out, int64_t n, void* s = nullptr) {
    return glmmoe_ref_silu_mul(g, u, out, n, s);
}

// cuda/kernels.cuh:63-66
inline int gemm_q(uint32_t qtype, const float* x, const uint8_t* qW, const float* bias, float* y,
                  int64_t n, int64_t in, int64_t out, int64_t row_bytes, void* s = nullptr) {
    return glmmoe_ref_gemm_q(qtype, x, qW, bias, y, n, in, out, row_bytes, s);
}

// cuda/kernels.cuh:117-123
inline int moe_expert_ffn_q(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                            const float* x, const int* topk_ids, const float* topk_w,
                            const uint8_t* gate_q, const uint8_t* up_q, const uint8_t* down_q,
                            int n, int topk, int hidden, int moe_inter, int E,
                            int64_t gate_row_bytes, int64_t up_row_bytes, int64_t down_row_bytes,
                            float* h_act, float* dpart, float* out, int* dispatch = nullptr,
                            float* gu_part = nullptr, void* s = nullptr) {
    return glmmoe_ref_moe_expert_ffn_q(gate_type, up_type, down_type, x, topk_ids, topk_w, gate_q,
                                       up_q, down_q, n, topk, hidden, moe_inter, E, gate_row_bytes,
                                       up_row_bytes, down_row_bytes, h_act, dpart, out, dispatch,
                                       gu_part, s);
}

// cuda/kernels.cuh:74-83
inline bool qtype_has_i8(uint32_t qtype) { return glmmoe_ref_qtype_has_i8(qtype) != 0; }
inline int quantize_act_q8(const float* x, int64_t n, int64_t in, int8_t* xq, float* xs,
                           void* s = nullptr) {
    return glmmoe_ref_quantize_act_q8(x, n, in, xq, xs, s);
}
inline int gemm_q_i8(uint32_t qtype, const int8_t* xq, const float* xs, const uint8_t* qW,
                     const float* bias, float* y, int64_t n, int64_t in, int64_t out,
                     int64_t row_bytes, void* s = nullptr) {
    return glmmoe_ref_gemm_q_i8(qtype, xq, xs, qW, bias, y, n, in, out, row_bytes, s);
}

// cuda/kernels.cuh:124-135
inline int moe_expert_ffn_q_i8(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                               const int8_t* xq, const float* xs, const int* topk_ids,
                               const float* topk_w, const uint8_t* gate_q, const uint8_t* up_q,
                               const uint8_t* down_q, int n, int topk, int hidden, int moe_inter,
                               int E, int64_t gate_row_bytes, int64_t up_row_bytes,
                               int64_t down_row_bytes, float* h_act, int8_t* hq, float* hs,
                               float* dpart, float* out, int* dispatch = nullptr,
                               float* gu_part = nullptr, void* s = nullptr) {
    return glmmoe_ref_moe_expert_ffn_q_i8(gate_type, up_type, down_type, xq, xs, topk_ids, topk_w,
                                          gate_q, up_q, down_q, n, topk, hidden, moe_inter, E,
                                          gate_row_bytes, up_row_bytes, down_row_bytes, h_act, hq,
                                          hs, dpart, out, dispatch, gu_part, s);
}

}  // namespace compat
}  // namespace glmmoe

#ifdef GLMMOE_GLMSERVE_NAMESPACE
namespace glmserve {
namespace cuda = ::glmmoe::compat;
}
#endif
