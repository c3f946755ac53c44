// Reference-signature C-ABI: the cuda/kernels.cuh launchers of the MoE branch
// (src/model_gpu.cpp:1448-1494) with the reference's arguments and fp32
// activations. Declarations and contracts: include/glmmoe.h.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <vector>

#include "../../include/glmmoe.h"
#include "kernels.hpp"

using namespace glmmoe;

namespace {

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Packed copies of reference-layout weight sets, keyed by the reference's
// qweight and scale pointers (host state; the lock covers lookups and
// updates). A call must name exactly a registered set: weights moved or
// replaced at other addresses are not found (GLMMOE_ERR_ARG) instead of
// silently using the old packed copy.
struct Registered {
    const uint8_t *gate_q, *up_q, *down_q;
    const float *gate_sc, *up_sc, *down_sc;
    glmmoe_w4a16_layer packed;
    bool same(const uint8_t* gq, const float* gs, const uint8_t* uq, const float* us,
              const uint8_t* dq, const float* ds) const {
        return gate_q == gq && up_q == uq && down_q == dq && gate_sc == gs && up_sc == us &&
               down_sc == ds;
    }
};
std::mutex g_mu;
std::vector<Registered> g_sets;
std::map<int, std::pair<void*, size_t>> g_ws;   // device -> caller workspace

// Routed-only layer descriptor of the given shape whose pointers are
// placeholders: used to size the workspace.
glmmoe_w4a16_layer shape_layer(int topk, int hidden, int moe_inter, int E) {
    glmmoe_w4a16_layer L{};
    L.hidden = hidden;
    L.moe_inter = moe_inter;
    L.n_experts = E;
    L.topk = topk;
    L.norm_topk = 1;
    L.routed_scale = 1.0f;
    const void* p = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));
    L.gate_q = L.up_q = L.down_q = static_cast<const uint8_t*>(p);
    L.gate_s = L.up_s = L.down_s = static_cast<const uint16_t*>(p);
    return L;
}

}  // namespace

extern "C" {

int glmmoe_ref_register_w4a16(const uint8_t* gate_q, const float* gate_sc, const uint8_t* up_q,
                              const float* up_sc, const uint8_t* down_q, const float* down_sc,
                              const glmmoe_w4a16_layer* packed) {
    if (!gate_q || !up_q || !down_q || !gate_sc || !up_sc || !down_sc || !packed)
        return GLMMOE_ERR_ARG;
    if (!packed->gate_q || !packed->gate_s || !packed->up_q || !packed->up_s ||
        !packed->down_q || !packed->down_s)
        return GLMMOE_ERR_ARG;
    Registered r{gate_q, up_q, down_q, gate_sc, up_sc, down_sc, *packed};
    // Routed experts only: the reference's moe_expert_ffn_w4a16 has no shared
    // expert and no router.
    r.packed.sh_gate_q = r.packed.sh_up_q = r.packed.sh_down_q = nullptr;
    r.packed.sh_gate_s = r.packed.sh_up_s = r.packed.sh_down_s = nullptr;
    r.packed.router_w = nullptr;
    r.packed.e_bias = nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto& e : g_sets)
        if (e.same(gate_q, gate_sc, up_q, up_sc, down_q, down_sc)) {
            e = r;
            return GLMMOE_OK;
        }
    g_sets.push_back(r);
    return GLMMOE_OK;
}

int glmmoe_ref_unregister_w4a16(const uint8_t* gate_q, const float* gate_sc, const uint8_t* up_q,
                                const float* up_sc, const uint8_t* down_q, const float* down_sc) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (size_t i = 0; i < g_sets.size(); ++i)
        if (g_sets[i].same(gate_q, gate_sc, up_q, up_sc, down_q, down_sc)) {
            g_sets.erase(g_sets.begin() + (long)i);
            return GLMMOE_OK;
        }
    return GLMMOE_ERR_ARG;
}

size_t glmmoe_ref_workspace_bytes(int n, int topk, int hidden, int moe_inter, int E) {
    if (n <= 0 || topk <= 0 || hidden <= 0 || moe_inter <= 0 || E <= 0) return 0;
    const glmmoe_w4a16_layer L = shape_layer(topk, hidden, moe_inter, E);
    const size_t lw = glmmoe_layer_workspace_bytes(&L, n);
    if (!lw) return 0;
    return align256((size_t)n * hidden * 2) + lw;
}

int glmmoe_ref_set_workspace(void* workspace, size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return GLMMOE_ERR_LAUNCH;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!workspace || !bytes) g_ws.erase(dev);
    else g_ws[dev] = {workspace, bytes};
    return GLMMOE_OK;
}

int glmmoe_ref_moe_expert_ffn_w4a16(const float* x, const int* topk_ids, const float* topk_weights,
                                    const uint8_t* gate_q, const float* gate_sc,
                                    const uint8_t* up_q, const float* up_sc,
                                    const uint8_t* down_q, const float* down_sc, int n, int topk,
                                    int hidden, int moe_inter, int E, int group_size, float* out,
                                    void* stream) {
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !topk_ids || !topk_weights || !out || n < 0) return GLMMOE_ERR_ARG;
    if (group_size != 128) return GLMMOE_ERR_SHAPE;
    glmmoe_w4a16_layer L;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        const Registered* hit = nullptr;
        for (const auto& e : g_sets)
            if (e.same(gate_q, gate_sc, up_q, up_sc, down_q, down_sc)) hit = &e;
        if (!hit) return GLMMOE_ERR_ARG;
        L = hit->packed;
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return GLMMOE_ERR_LAUNCH;
        const auto w = g_ws.find(dev);
        if (w == g_ws.end()) return GLMMOE_ERR_WORKSPACE;
        ws = w->second.first;
        ws_bytes = w->second.second;
    }
    if (L.hidden != hidden || L.moe_inter != moe_inter || L.n_experts != E) return GLMMOE_ERR_SHAPE;
    L.topk = topk;
    L.norm_topk = 1;        // unused: the weights come from the caller
    L.routed_scale = 1.0f;
    const size_t xb = align256((size_t)n * hidden * 2);
    const size_t need = glmmoe_ref_workspace_bytes(n, topk, hidden, moe_inter, E);
    if (!need) return GLMMOE_ERR_SHAPE;
    if (ws_bytes < need) return GLMMOE_ERR_WORKSPACE;
    uint16_t* xbf = static_cast<uint16_t*>(ws);
    int rc = launch_f32_to_bf16(x, xbf, (long)n * hidden, S(stream));
    if (rc) return GLMMOE_ERR_LAUNCH;
    return glmmoe_expert_ffn_w4a16(&L, xbf, n, topk_ids, topk_weights, out,
                                   static_cast<char*>(ws) + xb, ws_bytes - xb, stream);
}

int glmmoe_ref_moe_expert_ffn(const float* x, const int* topk_ids, const float* topk_weights,
                              const float* gate_w, const float* up_w, const float* down_w, int n,
                              int topk, int hidden, int moe_inter, int E, float* out,
                              void* stream) {
    (void)E;
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !topk_ids || !topk_weights || !gate_w || !up_w || !down_w || !out || n <= 0 ||
        topk <= 0 || hidden <= 0 || moe_inter <= 0)
        return GLMMOE_ERR_ARG;
    const int rc = launch_ref_expert_f32(x, topk_ids, topk_weights, gate_w, up_w, down_w, n, topk,
                                         hidden, moe_inter, out, S(stream));
    return rc == -2 ? GLMMOE_ERR_SHAPE : rc ? GLMMOE_ERR_LAUNCH : GLMMOE_OK;
}

int glmmoe_ref_gemm_w4a16(const float* x, const uint8_t* qW, const float* scales,
                          const float* bias, float* y, int64_t n, int64_t in, int64_t out,
                          int64_t group_size, void* stream) {
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !qW || !scales || !y || n <= 0 || in <= 0 || out <= 0 || group_size <= 0)
        return GLMMOE_ERR_ARG;
    if (n > INT32_MAX || in > INT32_MAX || out > INT32_MAX) return GLMMOE_ERR_SHAPE;
    return launch_ref_gemm_w4(x, qW, scales, bias, y, (int)n, (int)in, (int)out, (int)group_size,
                              S(stream))
               ? GLMMOE_ERR_LAUNCH
               : GLMMOE_OK;
}

int glmmoe_ref_gemm_fp8(const float* x, const uint8_t* fp8W, const float* w_scale,
                        const float* bias, float* y, int64_t n, int64_t in, int64_t out,
                        void* stream) {
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !fp8W || !y || n <= 0 || in <= 0 || out <= 0) return GLMMOE_ERR_ARG;
    if (n > INT32_MAX || in > INT32_MAX || out > INT32_MAX) return GLMMOE_ERR_SHAPE;
    return launch_ref_gemm_fp8(x, fp8W, w_scale, bias, y, (int)n, (int)in, (int)out, S(stream))
               ? GLMMOE_ERR_LAUNCH
               : GLMMOE_OK;
}

int glmmoe_ref_silu_mul(const float* g, const float* u, float* out, int64_t n, void* stream) {
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!g || !u || !out || n <= 0) return GLMMOE_ERR_ARG;
    return launch_ref_silu_mul(g, u, out, (long)n, S(stream)) ? GLMMOE_ERR_LAUNCH : GLMMOE_OK;
}

int glmmoe_ref_add_inplace(float* y, const float* x, int64_t n, void* stream) {
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!y || !x || n <= 0) return GLMMOE_ERR_ARG;
    return launch_ref_add_inplace(y, x, (long)n, S(stream)) ? GLMMOE_ERR_LAUNCH : GLMMOE_OK;
}

// Rows of `in` elements of GGUF type t fit row_bytes and decode 8 at a time.
static bool gguf_rows_ok(uint32_t t, int64_t in, int64_t row_bytes) {
    const int be = gguf_block_elems(t), bb = gguf_block_bytes(t);
    return be && in % be == 0 && in % 8 == 0 && row_bytes >= in / be * bb;
}

int glmmoe_ref_gemm_q(uint32_t qtype, const float* x, const uint8_t* qW, const float* bias,
                      float* y, int64_t n, int64_t in, int64_t out, int64_t row_bytes,
                      void* stream) {
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !qW || !y || n <= 0 || in <= 0 || out <= 0) return GLMMOE_ERR_ARG;
    if (n > INT32_MAX || in > INT32_MAX || out > INT32_MAX || !gguf_rows_ok(qtype, in, row_bytes))
        return GLMMOE_ERR_SHAPE;
    return launch_gg_gemm(qtype, x, qW, bias, y, (int)n, (int)in, (int)out, (long)row_bytes,
                          S(stream))
               ? GLMMOE_ERR_LAUNCH
               : GLMMOE_OK;
}

int glmmoe_ref_moe_expert_ffn_q(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                                const float* x, const int* topk_ids, const float* topk_w,
                                const uint8_t* gate_q, const uint8_t* up_q, const uint8_t* down_q,
                                int n, int topk, int hidden, int moe_inter, int E,
                                int64_t gate_row_bytes, int64_t up_row_bytes,
                                int64_t down_row_bytes, float* h_act, float* dpart, float* out,
                                int* dispatch, float* gu_part, void* stream) {
    (void)gu_part;   // split-K partials of the reference's decode path; not needed here
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !topk_ids || !topk_w || !gate_q || !up_q || !down_q || !h_act || !dpart || !out ||
        n <= 0 || topk <= 0 || hidden <= 0 || moe_inter <= 0 || E <= 0)
        return GLMMOE_ERR_ARG;
    if (E > 4096 || (int64_t)n * topk > INT32_MAX / 2 || !gguf_rows_ok(gate_type, hidden, gate_row_bytes) ||
        !gguf_rows_ok(up_type, hidden, up_row_bytes) ||
        !gguf_rows_ok(down_type, moe_inter, down_row_bytes))
        return GLMMOE_ERR_SHAPE;
    return launch_gg_moe(gate_type, up_type, down_type, x, topk_ids, topk_w, gate_q, up_q, down_q,
                         n, topk, hidden, moe_inter, E, (long)gate_row_bytes, (long)up_row_bytes,
                         (long)down_row_bytes, h_act, dpart, out, dispatch, S(stream))
               ? GLMMOE_ERR_LAUNCH
               : GLMMOE_OK;
}

int glmmoe_ref_qtype_has_i8(uint32_t qtype) { return gguf_has_i8(qtype) ? 1 : 0; }

int glmmoe_ref_quantize_act_q8(const float* x, int64_t n, int64_t in, int8_t* xq, float* xs,
                               void* stream) {
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !xq || !xs || n <= 0 || in <= 0) return GLMMOE_ERR_ARG;
    if (in % 32 || n > INT32_MAX || in > INT32_MAX) return GLMMOE_ERR_SHAPE;
    return launch_gg_quant_q8(x, (long)(n * in), xq, xs, S(stream)) ? GLMMOE_ERR_LAUNCH
                                                                   : GLMMOE_OK;
}

// int8 activation rows are read four bytes at a time.
static bool i8_rows_ok(const int8_t* q, int64_t in) {
    return in % 32 == 0 && ((uintptr_t)q & 3) == 0;
}

int glmmoe_ref_gemm_q_i8(uint32_t qtype, const int8_t* xq, const float* xs, const uint8_t* qW,
                         const float* bias, float* y, int64_t n, int64_t in, int64_t out,
                         int64_t row_bytes, void* stream) {
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!xq || !xs || !qW || !y || n <= 0 || in <= 0 || out <= 0) return GLMMOE_ERR_ARG;
    if (n > INT32_MAX || in > INT32_MAX || out > INT32_MAX || !gguf_has_i8(qtype) ||
        !gguf_rows_ok(qtype, in, row_bytes) || !i8_rows_ok(xq, in))
        return GLMMOE_ERR_SHAPE;
    return launch_gg_gemm_i8(qtype, xq, xs, qW, bias, y, (int)n, (int)in, (int)out,
                             (long)row_bytes, S(stream))
               ? GLMMOE_ERR_LAUNCH
               : GLMMOE_OK;
}

int glmmoe_ref_moe_expert_ffn_q_i8(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                                   const int8_t* xq, const float* xs, const int* topk_ids,
                                   const float* topk_w, const uint8_t* gate_q,
                                   const uint8_t* up_q, const uint8_t* down_q, int n, int topk,
                                   int hidden, int moe_inter, int E, int64_t gate_row_bytes,
                                   int64_t up_row_bytes, int64_t down_row_bytes, float* h_act,
                                   int8_t* hq, float* hs, float* dpart, float* out, int* dispatch,
                                   float* gu_part, void* stream) {
    (void)gu_part;
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!xq || !xs || !topk_ids || !topk_w || !gate_q || !up_q || !down_q || !h_act || !hq ||
        !hs || !dpart || !out || n <= 0 || topk <= 0 || hidden <= 0 || moe_inter <= 0 || E <= 0)
        return GLMMOE_ERR_ARG;
    if (E > 4096 || (int64_t)n * topk > INT32_MAX / 2 || !gguf_has_i8(gate_type) ||
        !gguf_has_i8(up_type) || !gguf_has_i8(down_type) ||
        !gguf_rows_ok(gate_type, hidden, gate_row_bytes) ||
        !gguf_rows_ok(up_type, hidden, up_row_bytes) ||
        !gguf_rows_ok(down_type, moe_inter, down_row_bytes) || !i8_rows_ok(xq, hidden) ||
        !i8_rows_ok(hq, moe_inter))
        return GLMMOE_ERR_SHAPE;
    return launch_gg_moe_i8(gate_type, up_type, down_type, xq, xs, topk_ids, topk_w, gate_q, up_q,
                            down_q, n, topk, hidden, moe_inter, E, (long)gate_row_bytes,
                            (long)up_row_bytes, (long)down_row_bytes, h_act, hq, hs, dpart, out,
                            dispatch, S(stream))
               ? GLMMOE_ERR_LAUNCH
               : GLMMOE_OK;
}

}  // extern "C"
