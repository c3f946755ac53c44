// ref_harness.cpp -- C entry points into the compiled glmserve reference CPU
// path, for the test suite and the CPU baseline ONLY (never the product).
//
// Compiled together with the reference's own sources (src/model_glm52.cpp and
// the files it links against) by oracle/Makefile into oracle/_ref/. No
// reference source is copied: the Makefile compiles them where they lie.
//
// GLM52Model::moe_mlp (src/model_glm52.cpp:1096-1154) is a private member
// (include/model.hpp:294); the harness reaches it by compiling its own
// translation unit with class access opened. Layout is unchanged by access
// specifiers, so the objects are the ones the reference builds.
#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>
#include <map>
#include <functional>
#include <stdexcept>

#define private public
#include "model.hpp"
#undef private
#include "tensor.hpp"
#include "gguf_quant.hpp"

using glmserve::GLM52Config;
using glmserve::GLM52Model;
using glmserve::Linear;
using glmserve::MoEMLP;

static void fill_linear(Linear& L, const float* w, int64_t out, int64_t in) {
    L.out_features = out;
    L.in_features = in;
    if (w) L.w.assign(w, w + out * in);
}

extern "C" {

// hw_threads(): src/model_glm52.cpp:21-24 (min(hardware_concurrency, 32)).
int ref_hw_threads() {
    unsigned n = std::thread::hardware_concurrency();
    return (int)(n == 0 ? 1u : std::min(n, 32u));
}
int ref_hardware_concurrency() { return (int)std::thread::hardware_concurrency(); }

// src/tensor.cpp:53-63.
void ref_dequant_int4(const uint8_t* packed, const float* scales, int64_t count,
                      int64_t group_size, float* out) {
    glmserve::dequant_int4_to_f32(packed, scales, count, group_size, out);
}

// Runs the reference GLM52Model::moe_mlp once over n tokens. Experts whose
// gate pointer is NULL are left empty (the reference aborts via GLM_CHECK if
// routing selects one). sh_* may be NULL (no shared expert). If seconds is
// non-NULL it receives the wall time of the moe_mlp call alone (weight copies
// into the reference's containers are excluded). Returns 0, -1 on exception.
int ref_moe_mlp(const float* x, int64_t n, int64_t H, int E, int topk, int64_t I, int64_t S,
                const float* router_w, const float* e_bias, const float* const* gate,
                const float* const* up, const float* const* down, const float* sh_gate,
                const float* sh_up, const float* sh_down, int norm_topk, double routed_scale,
                float* out, double* seconds) {
    try {
        GLM52Config cfg;
        cfg.hidden_size = H;
        cfg.n_routed_experts = E;
        cfg.num_experts_per_tok = topk;
        cfg.moe_intermediate_size = I;
        cfg.norm_topk_prob = norm_topk != 0;
        cfg.routed_scaling_factor = routed_scale;
        GLM52Model model(cfg);
        MoEMLP m;
        fill_linear(m.router, router_w, E, H);
        if (e_bias) m.e_bias.assign(e_bias, e_bias + E);
        m.experts.resize(E);
        for (int e = 0; e < E; ++e) {
            if (!gate[e]) continue;
            fill_linear(m.experts[e].gate_proj, gate[e], I, H);
            fill_linear(m.experts[e].up_proj, up[e], I, H);
            fill_linear(m.experts[e].down_proj, down[e], H, I);
        }
        if (sh_gate) {
            m.has_shared = true;
            fill_linear(m.shared.gate_proj, sh_gate, S, H);
            fill_linear(m.shared.up_proj, sh_up, S, H);
            fill_linear(m.shared.down_proj, sh_down, H, S);
        }
        auto t0 = std::chrono::steady_clock::now();
        model.moe_mlp(m, x, out, n);
        auto t1 = std::chrono::steady_clock::now();
        if (seconds) *seconds = std::chrono::duration<double>(t1 - t0).count();
        return 0;
    } catch (...) {
        return -1;
    }
}

// src/gguf_quant.cpp: one row of n elements of a GGUF tensor (row 0 of data).
// Returns 0, -1 for a type it cannot dequantize.
int ref_gguf_dequant_row(uint32_t type, const uint8_t* data, int64_t n, float* out) {
    if (!glmserve::gguf_type_can_dequantize(type)) return -1;
    const std::vector<float> v = glmserve::gguf_dequantize_row(type, data, (uint64_t)n, 0);
    std::memcpy(out, v.data(), (size_t)n * sizeof(float));
    return 0;
}

// The reference's dequant codebooks (src/gguf_quant.cpp:363-381).
void ref_gguf_tables(const uint8_t** iq3xxs_grid, const uint8_t** ksigns, const int8_t** iq4nl) {
    *iq3xxs_grid = glmserve::gguf_iq3xxs_grid_table();
    *ksigns = glmserve::gguf_ksigns_iq2xs_table();
    *iq4nl = glmserve::gguf_kvalues_iq4nl_table();
}

}  // extern "C"
