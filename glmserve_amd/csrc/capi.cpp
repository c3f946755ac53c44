// C-ABI of the MoE-layer hot path: argument checks, workspace carving and the
// launch sequence. Declarations and contracts: include/glmmoe.h.
#include <hip/hip_runtime.h>

#include "../../include/glmmoe.h"
#include "kernels.hpp"

using namespace glmmoe;

namespace {

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

constexpr int kStreamWeightsMinTokens = 2;   // non-temporal expert-weight loads from this batch

// Tile height of the W4A16 expert GEMMs for a batch: 16-row tiles (decode
// kernels) or, from kBigMinRows grouped rows on shapes the large-group kernels
// take (both K-group counts multiples of 8), 128-row tiles.
inline int tile_rows_for(int n, int topk, int with_shared, int H, int I) {
    return (long)n * topk + (with_shared ? n : 0) >= kBigMinRows && big_w4_shape_ok(H, I)
               ? kBigRows
               : kTileRows;
}

int max_tiles_for(int n, int topk, int E, int with_shared, int T) {
    // sum_e ceil(c_e / T) <= (n*topk)/T + E, plus ceil(n/T) shared tiles.
    return (n * topk) / T + E + (with_shared ? (n + T - 1) / T : 0) + 1;
}

int max_tiles_for(int n, int topk, int E, int with_shared, int H, int I) {
    return max_tiles_for(n, topk, E, with_shared, tile_rows_for(n, topk, with_shared, H, I));
}

// Shape and pointer checks shared by the W4A16 and FP8 layer descriptors.
template <class Layer>
int check_layer(const Layer* L, int n) {
    if (!L || n < 0) return GLMMOE_ERR_ARG;
    if (L->hidden <= 0 || L->moe_inter <= 0 || L->n_experts <= 0 || L->topk <= 0)
        return GLMMOE_ERR_ARG;
    if (L->hidden % 256 || L->moe_inter % 128 || L->hidden > 8192) return GLMMOE_ERR_SHAPE;
    if (L->n_experts > 512 || L->topk > 8 || L->topk > L->n_experts) return GLMMOE_ERR_SHAPE;
    if (!L->gate_q || !L->gate_s || !L->up_q || !L->up_s || !L->down_q || !L->down_s)
        return GLMMOE_ERR_ARG;
    const bool any_sh = L->sh_gate_q || L->sh_up_q || L->sh_down_q;
    const bool all_sh = L->sh_gate_q && L->sh_gate_s && L->sh_up_q && L->sh_up_s &&
                        L->sh_down_q && L->sh_down_s;
    if (any_sh && !all_sh) return GLMMOE_ERR_ARG;
    return GLMMOE_OK;
}

template <class Layer>
inline bool has_shared(const Layer* L) { return L->sh_gate_q != nullptr; }

ExpertPtrs ptrs(const glmmoe_w4a16_layer* L) {
    return ExpertPtrs{L->gate_q, L->gate_s, L->up_q, L->up_s, L->down_q, L->down_s,
                      L->sh_gate_q, L->sh_gate_s, L->sh_up_q, L->sh_up_s, L->sh_down_q,
                      L->sh_down_s};
}

// The router scratch is free once routing is done; a large batch's dispatch
// uses it for its chunk histograms (when it is large enough).
template <class Layer>
int* dispatch_scratch(float* rpart, const Layer* L, int n) {
    const size_t need = dispatch_scratch_bytes(n, L->topk, L->n_experts);
    if (!need || router_select_scratch_bytes(n, L->hidden, L->n_experts) < need) return nullptr;
    return reinterpret_cast<int*>(rpart);
}

// Bytes of the dpart region: the per-row expert outputs, and before them (it
// is free while the gate/up kernel runs) the partials of the gate/up stream
// kernel's split items: up to kTailTicks items of H / 2048 parts of 16 KiB.
size_t dpart_bytes(const glmmoe_w4a16_layer* L, int n) {
    const size_t R = (size_t)n * L->topk + (has_shared(L) ? (size_t)n : 0);
    const size_t rows = R * L->hidden * 4;
    const size_t tail = (size_t)kTailTicks * (L->hidden / 2048) * 16384;
    return rows > tail ? rows : tail;
}

// Carves the workspace; with base == nullptr only computes the size.
size_t carve(const glmmoe_w4a16_layer* L, int n, char* base, glmmoe_layer_ws* v) {
    const int H = L->hidden, I = L->moe_inter, E = L->n_experts, k = L->topk;
    const size_t nk = (size_t)n * k;
    const size_t R = nk + (has_shared(L) ? (size_t)n : 0);
    const size_t mt = (size_t)max_tiles_for(n, k, E, has_shared(L), H, I);
    size_t off = 0;
    auto take = [&](size_t bytes) -> char* {
        char* p = base ? base + off : nullptr;
        off += align256(bytes);
        return p;
    };
    glmmoe_layer_ws w{};
    w.logits = reinterpret_cast<float*>(take((size_t)n * E * 4));
    w.rpart = reinterpret_cast<float*>(take(router_select_scratch_bytes(n, H, E)));
    w.xsum = reinterpret_cast<float*>(take((size_t)n * (H / 128) * 4));
    w.topk_ids = reinterpret_cast<int*>(take(nk * 4));
    w.topk_w = reinterpret_cast<float*>(take(nk * 4));
    w.expert_offsets = reinterpret_cast<int*>(take((size_t)(E + 2) * 4));
    w.sorted_token_ids = reinterpret_cast<int*>(take(R * 4));
    w.sorted_row = reinterpret_cast<int*>(take(R * 4));
    w.inv = reinterpret_cast<int*>(take(nk * 4));
    w.tiles = reinterpret_cast<int*>(take(mt * 16));
    w.ntiles = reinterpret_cast<int*>(take(16));
    w.h = reinterpret_cast<uint16_t*>(take(R * I * 2));
    w.hsum = reinterpret_cast<float*>(take(R * (I / 128) * 4));
    w.dpart = reinterpret_cast<float*>(take(dpart_bytes(L, n)));
    w.sync = reinterpret_cast<unsigned int*>(take(kTailTicks * 4));
    w.bytes = off;
    if (v) *v = w;
    return off;
}

Fp8Ptrs ptrs8(const glmmoe_fp8_layer* L) {
    return Fp8Ptrs{L->gate_q, L->gate_s, L->up_q, L->up_s, L->down_q, L->down_s,
                   L->sh_gate_q, L->sh_gate_s, L->sh_up_q, L->sh_up_s, L->sh_down_q,
                   L->sh_down_s};
}

size_t carve8(const glmmoe_fp8_layer* L, int n, char* base, glmmoe_fp8_ws* v) {
    const int H = L->hidden, I = L->moe_inter, E = L->n_experts, k = L->topk;
    const size_t nk = (size_t)n * k;
    const size_t R = nk + (has_shared(L) ? (size_t)n : 0);
    const size_t mt = (size_t)max_tiles_for(n, k, E, has_shared(L), kBigRows);
    size_t off = 0;
    auto take = [&](size_t bytes) -> char* {
        char* p = base ? base + off : nullptr;
        off += align256(bytes);
        return p;
    };
    glmmoe_fp8_ws w{};
    w.logits = reinterpret_cast<float*>(take((size_t)n * E * 4));
    w.rpart = reinterpret_cast<float*>(take(router_select_scratch_bytes(n, H, E)));
    w.xq = reinterpret_cast<uint8_t*>(take((size_t)n * H));
    w.xscale = reinterpret_cast<float*>(take((size_t)n * (H / 128) * 4));
    w.topk_ids = reinterpret_cast<int*>(take(nk * 4));
    w.topk_w = reinterpret_cast<float*>(take(nk * 4));
    w.expert_offsets = reinterpret_cast<int*>(take((size_t)(E + 2) * 4));
    w.sorted_token_ids = reinterpret_cast<int*>(take(R * 4));
    w.sorted_row = reinterpret_cast<int*>(take(R * 4));
    w.inv = reinterpret_cast<int*>(take(nk * 4));
    w.tiles = reinterpret_cast<int*>(take(mt * 16));
    w.ntiles = reinterpret_cast<int*>(take(16));
    w.hq = reinterpret_cast<uint8_t*>(take(R * I));
    w.hscale = reinterpret_cast<float*>(take(R * (I / 128) * 4));
    w.dpart = reinterpret_cast<float*>(take(R * H * 4));
    w.bytes = off;
    if (v) *v = w;
    return off;
}

// ---- stage timing ring ------------------------------------------------------
struct Prof {
    bool on = false;
    bool created = false;
    int calls = 0;                       // calls recorded since the last read
    hipEvent_t ev[GLMMOE_PROF_MAX_CALLS][GLMMOE_N_STAGES + 1];
    bool has[GLMMOE_PROF_MAX_CALLS][GLMMOE_N_STAGES + 1];
};
Prof g_prof;

// Records the boundary before stage `stage` (stage == N_STAGES: after the last).
inline void mark(int stage, hipStream_t s) {
    if (!g_prof.on || g_prof.calls >= GLMMOE_PROF_MAX_CALLS) return;
    (void)hipEventRecord(g_prof.ev[g_prof.calls][stage], s);
    g_prof.has[g_prof.calls][stage] = true;
}
inline void begin_call() {
    if (!g_prof.on || g_prof.calls >= GLMMOE_PROF_MAX_CALLS) return;
    for (int i = 0; i <= GLMMOE_N_STAGES; ++i) g_prof.has[g_prof.calls][i] = false;
}
inline void end_call(hipStream_t s) {
    if (!g_prof.on || g_prof.calls >= GLMMOE_PROF_MAX_CALLS) return;
    mark(GLMMOE_N_STAGES, s);
    ++g_prof.calls;
}

// Dispatch onward, given ids/weights/xsum in the workspace view.
// x16_ready: the router already wrote x's fp16 rows for the large-group
// gate/up kernel into the start of dpart.
int run_experts(const glmmoe_w4a16_layer* L, const uint16_t* x, int n, const int* ids,
                const float* w, const float* xsum, float* out, const glmmoe_layer_ws& v,
                hipStream_t s, bool dispatched = false, const FusedRoute* fr = nullptr,
                bool x16_ready = false) {
    const int H = L->hidden, I = L->moe_inter, E = L->n_experts, k = L->topk;
    const int sh = has_shared(L) ? 1 : 0;
    const int mt = max_tiles_for(n, k, E, sh, H, I);
    const int T = tile_rows_for(n, k, sh, H, I);
    const bool big = T == kBigRows;
    mark(GLMMOE_STAGE_DISPATCH, s);
    int rc = dispatched || fr ? 0
                        : launch_dispatch(ids, n, k, E, v.expert_offsets, v.sorted_token_ids,
                                          v.sorted_row, v.inv, v.tiles, v.ntiles, T, sh, 1, s,
                                          dispatch_scratch(v.rpart, L, n), big ? kBigRows / 2 : 0,
                                          v.sync, kTailTicks);
    if (rc) return rc;
    const ExpertPtrs P = ptrs(L);
    // From two tokens the routed experts' weights (up to 2 * topk + 1 of
    // them) outgrow the 256 MiB Infinity Cache: stream them past L2.
    const bool nt = n >= kStreamWeightsMinTokens;
    mark(GLMMOE_STAGE_GATE_UP, s);
    // The large-group path keeps h's block exponents where the decode
    // kernels keep h's group sums (I / 32 bytes per row either way).
    int8_t* hexp = reinterpret_cast<int8_t*>(v.hsum);
    const int R = n * k + sh * n;
    rc = big ? launch_gate_up_big(P, x, n, v.tiles, v.ntiles, mt, v.sorted_token_ids, v.h, hexp, v.dpart,
                                  dpart_bytes(L, n), v.sync, H, I, E, s, x16_ready)
             : launch_gate_up(P, x, xsum, v.tiles, v.ntiles, mt, v.sorted_token_ids, v.h, v.hsum,
                              v.sync, v.dpart, dpart_bytes(L, n), H, I, E, s, fr, nt);
    if (rc) return rc;
    mark(GLMMOE_STAGE_DOWN, s);
    rc = big ? launch_down_big(P, v.h, hexp, R, v.tiles, v.ntiles, mt, v.dpart, H, I, E, s)
             : launch_down(P, v.h, v.hsum, v.tiles, v.ntiles, mt, v.dpart, H, I, E, s, nt);
    if (rc) return rc;
    mark(GLMMOE_STAGE_COMBINE, s);
    rc = launch_combine(v.dpart, v.inv, w, n, k, H, sh, out, s, big);
    if (rc) return rc;
    end_call(s);
    return GLMMOE_OK;
}

// FP8: activation quantization, dispatch onto 128-row tiles, the two fp8
// grouped GEMMs and the combine.
int run_experts8(const glmmoe_fp8_layer* L, const uint16_t* x, int n, const int* ids,
                 const float* w, float* out, const glmmoe_fp8_ws& v, hipStream_t s,
                 bool dispatched = false) {
    const int H = L->hidden, I = L->moe_inter, E = L->n_experts, k = L->topk;
    const int sh = has_shared(L) ? 1 : 0;
    const int mt = max_tiles_for(n, k, E, sh, kBigRows);
    int rc = launch_quant_act_fp8(x, n, H, v.xq, v.xscale, s);
    if (rc) return rc;
    mark(GLMMOE_STAGE_DISPATCH, s);
    rc = dispatched ? 0
                    : launch_dispatch(ids, n, k, E, v.expert_offsets, v.sorted_token_ids,
                                      v.sorted_row, v.inv, v.tiles, v.ntiles, kBigRows, sh, 1, s,
                                      dispatch_scratch(v.rpart, L, n));
    if (rc) return rc;
    const Fp8Ptrs P = ptrs8(L);
    mark(GLMMOE_STAGE_GATE_UP, s);
    rc = launch_gate_up_fp8(P, v.xq, v.xscale, v.tiles, v.ntiles, mt, v.sorted_token_ids, v.hq,
                            v.hscale, H, I, E, s);
    if (rc) return rc;
    mark(GLMMOE_STAGE_DOWN, s);
    rc = launch_down_fp8(P, v.hq, v.hscale, v.tiles, v.ntiles, mt, v.dpart, H, I, E, s);
    if (rc) return rc;
    mark(GLMMOE_STAGE_COMBINE, s);
    rc = launch_combine(v.dpart, v.inv, w, n, k, H, sh, out, s, true);
    if (rc) return rc;
    end_call(s);
    return GLMMOE_OK;
}

}  // namespace

extern "C" {

const char* glmmoe_version(void) { return "glmmoe 0.1 (gfx950)"; }

size_t glmmoe_router_logits_workspace_bytes(int n, int H, int E) {
    if (n <= 0 || H <= 0 || E <= 0) return 0;   // n == 0: no workspace needed
    return router_logits_scratch_bytes(n, H, E);
}

int glmmoe_router_logits(const uint16_t* x, const uint16_t* wr, int n, int H, int E,
                         float* logits, float* xsum, void* workspace, size_t workspace_bytes,
                         void* stream) {
    if (n == 0 && H > 0 && E > 0) return GLMMOE_OK;
    if (!x || !wr || !logits || n <= 0 || H <= 0 || E <= 0) return GLMMOE_ERR_ARG;
    if (H % 8 || H > 8192) return GLMMOE_ERR_SHAPE;
    if (xsum && H % 128) return GLMMOE_ERR_SHAPE;
    const size_t need = router_logits_scratch_bytes(n, H, E);
    if (need && (!workspace || workspace_bytes < need)) return GLMMOE_ERR_WORKSPACE;
    return launch_router_logits(x, wr, n, H, E, logits, xsum, static_cast<float*>(workspace),
                                S(stream));
}

int glmmoe_router_logits_f32(const float* x, const float* W, const float* bias, float* y,
                             int64_t n, int64_t in, int64_t out, void* stream) {
    if (n == 0 && in > 0 && out > 0) return GLMMOE_OK;
    if (!x || !W || !y || n <= 0 || in <= 0 || out <= 0) return GLMMOE_ERR_ARG;
    if (in % 128 || in > 8192 || n > (1 << 30) || out > (1 << 20)) return GLMMOE_ERR_SHAPE;
    return launch_router_logits_f32(x, W, bias, y, (int)n, (int)in, (int)out, S(stream)) ? GLMMOE_ERR_LAUNCH
                                                                                         : GLMMOE_OK;
}

int glmmoe_moe_router(const float* logits, const float* e_bias, int n, int E, int topk,
                      int norm_topk, float routed_scale, int* topk_ids, float* topk_weights,
                      void* stream) {
    if (n == 0 && E > 0 && topk > 0) return GLMMOE_OK;
    if (!logits || !topk_ids || !topk_weights || n <= 0 || E <= 0 || topk <= 0)
        return GLMMOE_ERR_ARG;
    if (topk > 8 || topk > E || E > 512) return GLMMOE_ERR_SHAPE;
    return launch_router_topk(logits, e_bias, n, E, topk, norm_topk, routed_scale, topk_ids,
                              topk_weights, S(stream));
}

int glmmoe_moe_dispatch(const int* topk_ids, int n, int topk, int E, int* expert_offsets,
                        int* sorted_token_ids, int* sorted_row, void* stream) {
    // n == 0 still writes expert_offsets (all zero), as the reference's
    // kernel does (cuda/moe_dispatch.cu:23-26).
    if (!expert_offsets || n < 0 || topk <= 0 || E <= 0) return GLMMOE_ERR_ARG;
    if (n > 0 && (!topk_ids || !sorted_token_ids || !sorted_row)) return GLMMOE_ERR_ARG;
    if (E > 512 || (long)n * topk > (1L << 24)) return GLMMOE_ERR_SHAPE;
    return launch_dispatch(topk_ids, n, topk, E, expert_offsets, sorted_token_ids, sorted_row,
                           nullptr, nullptr, nullptr, kTileRows, 0, 0, S(stream));
}

size_t glmmoe_w4_packed_bytes(int rows, int K) { return (size_t)rows * K / 2; }
size_t glmmoe_w4_packed_scale_bytes(int rows, int K) { return (size_t)rows * (K / 128) * 2; }

int glmmoe_pack_w4a16(const uint8_t* qweight, const void* scales, int scales_dtype, int n_mats,
                      int rows, int K, int group_size, uint8_t* packed_q,
                      uint16_t* packed_scales, void* stream) {
    if (!qweight || !scales || !packed_q || !packed_scales || n_mats <= 0 || rows <= 0 ||
        K <= 0)
        return GLMMOE_ERR_ARG;
    if (rows % 16 || K % 128 || group_size != 128) return GLMMOE_ERR_SHAPE;
    if (scales_dtype != 0 && scales_dtype != 1) return GLMMOE_ERR_ARG;
    return launch_pack_w4(qweight, scales, scales_dtype, n_mats, rows, K, packed_q,
                          packed_scales, S(stream));
}

size_t glmmoe_layer_workspace_bytes(const glmmoe_w4a16_layer* L, int n) {
    if (check_layer(L, n)) return 0;
    return carve(L, n, nullptr, nullptr);
}

int glmmoe_layer_workspace_view(const glmmoe_w4a16_layer* L, int n, void* workspace,
                                glmmoe_layer_ws* view) {
    const int rc = check_layer(L, n);
    if (rc) return rc;
    if (!workspace || !view) return GLMMOE_ERR_ARG;
    carve(L, n, static_cast<char*>(workspace), view);
    return GLMMOE_OK;
}

}  // extern "C"

namespace {

// The MoE branch on a carved workspace. xf (fp32 activations) non-null: the
// bf16 rows x are written to xb first -- by the router kernel of the
// small-batch path as it stages them, otherwise by one conversion launch --
// and x is ignored.
int layer_w4(const glmmoe_w4a16_layer* L, const uint16_t* x, const float* xf, uint16_t* xb, int n,
             float* out, const glmmoe_layer_ws& v, hipStream_t s) {
    int rc = 0;
    const int H = L->hidden, E = L->n_experts, k = L->topk;
    begin_call();
    mark(GLMMOE_STAGE_ROUTER_LOGITS, s);
    if (xf) {
        if (!router_small_path(n, H, E, k)) {
            rc = launch_f32_to_bf16(xf, xb, (long)n * H, s);
            if (rc) return GLMMOE_ERR_LAUNCH;
            xf = nullptr;
        }
        x = xb;
    }
    // The router pass also writes the activation group sums the expert
    // kernels use to remove the int4 decode offset.
    const int sh = has_shared(L) ? 1 : 0;
    const int T = tile_rows_for(n, k, sh, H, L->moe_inter);
    const DispOut disp{v.expert_offsets, v.sorted_token_ids, v.sorted_row, v.inv,
                       reinterpret_cast<int4*>(v.tiles), v.ntiles, T, sh, 1,
                       T == kBigRows ? kBigRows / 2 : 0, v.sync, kTailTicks};
    // Small batches: the router kernel writes the order codes and scores,
    // and the gate/up kernel selects and dispatches (one launch fewer).
    if (T == kTileRows && router_small_path(n, H, E, k) && fused_route_ok(n, k, E, H)) {
        rc = launch_router_select(x, L->router_w, L->e_bias, n, H, E, k, L->norm_topk,
                                  L->routed_scale, v.logits, v.xsum, v.rpart, v.topk_ids, v.topk_w,
                                  s, &disp, nullptr, false, xf, xb);
        if (rc) return rc;
        mark(GLMMOE_STAGE_ROUTER_TOPK, s);
        const FusedRoute fr{reinterpret_cast<const uint32_t*>(v.rpart), n, k, L->norm_topk,
                            L->routed_scale, v.topk_ids, v.topk_w, disp};
        return run_experts(L, x, n, v.topk_ids, v.topk_w, v.xsum, out, v, s, true, &fr);
    }
    bool dispatched = false, x16 = false;
    // The large-group kernels do not read the activation group sums; their
    // fp16 input rows go to the start of dpart (launch_gate_up_big's scratch,
    // free until then) when the router stages whole rows.
    const bool big = T == kBigRows;
    uint16_t* xh = big ? reinterpret_cast<uint16_t*>(v.dpart) : nullptr;
    float* xrho = big ? reinterpret_cast<float*>(xh + (size_t)n * H) : nullptr;
    rc = launch_router_select(x, L->router_w, L->e_bias, n, H, E, k, L->norm_topk,
                              L->routed_scale, v.logits, big ? nullptr : v.xsum, v.rpart,
                              v.topk_ids, v.topk_w, s, &disp, &dispatched, true, xf, xb, xh, xrho,
                              &x16);
    if (rc) return rc;
    mark(GLMMOE_STAGE_ROUTER_TOPK, s);
    return run_experts(L, x, n, v.topk_ids, v.topk_w, v.xsum, out, v, s, dispatched, nullptr, x16);
}

}  // namespace

extern "C" {

int glmmoe_moe_layer_w4a16(const glmmoe_w4a16_layer* L, const uint16_t* x, int n, float* out,
                           void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_layer(L, n);
    if (rc) return rc;
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !out || !workspace || !L->router_w) return GLMMOE_ERR_ARG;
    glmmoe_layer_ws v;
    if (carve(L, n, static_cast<char*>(workspace), &v) > workspace_bytes)
        return GLMMOE_ERR_WORKSPACE;
    return layer_w4(L, x, nullptr, nullptr, n, out, v, S(stream));
}

size_t glmmoe_layer_f32_workspace_bytes(const glmmoe_w4a16_layer* L, int n) {
    if (check_layer(L, n)) return 0;
    return carve(L, n, nullptr, nullptr) + align256((size_t)n * L->hidden * 2);
}

int glmmoe_moe_layer_w4a16_f32(const glmmoe_w4a16_layer* L, const float* x, int n, float* out,
                               void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_layer(L, n);
    if (rc) return rc;
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !out || !workspace || !L->router_w) return GLMMOE_ERR_ARG;
    glmmoe_layer_ws v;
    const size_t lb = carve(L, n, static_cast<char*>(workspace), &v);
    if (lb + align256((size_t)n * L->hidden * 2) > workspace_bytes) return GLMMOE_ERR_WORKSPACE;
    uint16_t* xb = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + lb);
    return layer_w4(L, nullptr, x, xb, n, out, v, S(stream));
}

int glmmoe_moe_route_w4a16(const glmmoe_w4a16_layer* L, const uint16_t* x, int n,
                           int* topk_ids, float* topk_w, void* workspace,
                           size_t workspace_bytes, void* stream) {
    int rc = check_layer(L, n);
    if (rc) return rc;
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !topk_ids || !topk_w || !workspace || !L->router_w) return GLMMOE_ERR_ARG;
    glmmoe_layer_ws v;
    if (carve(L, n, static_cast<char*>(workspace), &v) > workspace_bytes)
        return GLMMOE_ERR_WORKSPACE;
    return launch_router_select(x, L->router_w, L->e_bias, n, L->hidden, L->n_experts, L->topk,
                                L->norm_topk, L->routed_scale, v.logits, v.xsum, v.rpart,
                                topk_ids, topk_w, S(stream));
}

int glmmoe_expert_ffn_w4a16(const glmmoe_w4a16_layer* L, const uint16_t* x, int n,
                            const int* topk_ids, const float* topk_w, float* out,
                            void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_layer(L, n);
    if (rc) return rc;
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !out || !workspace || !topk_ids || !topk_w) return GLMMOE_ERR_ARG;
    glmmoe_layer_ws v;
    if (carve(L, n, static_cast<char*>(workspace), &v) > workspace_bytes)
        return GLMMOE_ERR_WORKSPACE;
    hipStream_t s = S(stream);
    begin_call();
    mark(GLMMOE_STAGE_ROUTER_LOGITS, s);
    // The activation group sums are read only by the decode kernels (the
    // large-group kernels decode the int4 weights exactly instead).
    const int sh = has_shared(L) ? 1 : 0;
    if (tile_rows_for(n, L->topk, sh, L->hidden, L->moe_inter) != kBigRows) {
        rc = launch_xsum(x, n, L->hidden, v.xsum, s);
        if (rc) return rc;
    }
    return run_experts(L, x, n, topk_ids, topk_w, v.xsum, out, v, s);
}

size_t glmmoe_fp8_packed_bytes(int rows, int K) { return (size_t)rows * K; }

int glmmoe_pack_fp8(const uint8_t* w, int n_mats, int rows, int K, uint8_t* packed,
                    void* stream) {
    if (!w || !packed || n_mats <= 0 || rows <= 0 || K <= 0) return GLMMOE_ERR_ARG;
    if (rows % 128 || K % 128) return GLMMOE_ERR_SHAPE;
    return launch_pack_fp8(w, n_mats, rows, K, packed, S(stream));
}

int glmmoe_quant_act_fp8(const uint16_t* x, int n, int K, uint8_t* q, float* scale,
                         void* stream) {
    if (n == 0 && K > 0) return GLMMOE_OK;
    if (!x || !q || !scale || n <= 0 || K <= 0) return GLMMOE_ERR_ARG;
    if (K % 128) return GLMMOE_ERR_SHAPE;
    return launch_quant_act_fp8(x, n, K, q, scale, S(stream));
}

size_t glmmoe_fp8_layer_workspace_bytes(const glmmoe_fp8_layer* L, int n) {
    if (check_layer(L, n)) return 0;
    return carve8(L, n, nullptr, nullptr);
}

int glmmoe_fp8_layer_workspace_view(const glmmoe_fp8_layer* L, int n, void* workspace,
                                    glmmoe_fp8_ws* view) {
    const int rc = check_layer(L, n);
    if (rc) return rc;
    if (!workspace || !view) return GLMMOE_ERR_ARG;
    carve8(L, n, static_cast<char*>(workspace), view);
    return GLMMOE_OK;
}

int glmmoe_moe_layer_fp8(const glmmoe_fp8_layer* L, const uint16_t* x, int n, float* out,
                         void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_layer(L, n);
    if (rc) return rc;
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !out || !workspace || !L->router_w) return GLMMOE_ERR_ARG;
    glmmoe_fp8_ws v;
    if (carve8(L, n, static_cast<char*>(workspace), &v) > workspace_bytes)
        return GLMMOE_ERR_WORKSPACE;
    hipStream_t s = S(stream);
    const int H = L->hidden, E = L->n_experts, k = L->topk;
    begin_call();
    mark(GLMMOE_STAGE_ROUTER_LOGITS, s);
    const int sh = has_shared(L) ? 1 : 0;
    const DispOut disp{v.expert_offsets, v.sorted_token_ids, v.sorted_row, v.inv,
                       reinterpret_cast<int4*>(v.tiles), v.ntiles, kBigRows, sh, 1, 0, nullptr, 0};
    bool dispatched = false;
    rc = launch_router_select(x, L->router_w, L->e_bias, n, H, E, k, L->norm_topk,
                              L->routed_scale, v.logits, nullptr, v.rpart, v.topk_ids, v.topk_w, s,
                              &disp, &dispatched);
    if (rc) return rc;
    mark(GLMMOE_STAGE_ROUTER_TOPK, s);
    return run_experts8(L, x, n, v.topk_ids, v.topk_w, out, v, s, dispatched);
}

int glmmoe_expert_ffn_fp8(const glmmoe_fp8_layer* L, const uint16_t* x, int n,
                          const int* topk_ids, const float* topk_w, float* out,
                          void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_layer(L, n);
    if (rc) return rc;
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    if (!x || !out || !workspace || !topk_ids || !topk_w) return GLMMOE_ERR_ARG;
    glmmoe_fp8_ws v;
    if (carve8(L, n, static_cast<char*>(workspace), &v) > workspace_bytes)
        return GLMMOE_ERR_WORKSPACE;
    begin_call();
    mark(GLMMOE_STAGE_ROUTER_LOGITS, S(stream));   // the activation quantization
    return run_experts8(L, x, n, topk_ids, topk_w, out, v, S(stream));
}

int glmmoe_profile_enable(int on) {
    if (on && !g_prof.created) {
        for (int c = 0; c < GLMMOE_PROF_MAX_CALLS; ++c)
            for (int i = 0; i <= GLMMOE_N_STAGES; ++i)
                if (hipEventCreate(&g_prof.ev[c][i]) != hipSuccess) return GLMMOE_ERR_LAUNCH;
        g_prof.created = true;
    }
    g_prof.on = on != 0;
    g_prof.calls = 0;
    return GLMMOE_OK;
}

int glmmoe_profile_read(float* stage_ms, int* n_calls) {
    if (!stage_ms || !n_calls) return GLMMOE_ERR_ARG;
    for (int i = 0; i < GLMMOE_N_STAGES; ++i) { stage_ms[i] = 0.0f; n_calls[i] = 0; }
    for (int c = 0; c < g_prof.calls; ++c) {
        if (hipEventSynchronize(g_prof.ev[c][GLMMOE_N_STAGES]) != hipSuccess)
            return GLMMOE_ERR_LAUNCH;
        // Each recorded stage runs from its mark to the next recorded mark.
        for (int i = 0; i < GLMMOE_N_STAGES; ++i) {
            if (!g_prof.has[c][i]) continue;
            int j = i + 1;
            while (j <= GLMMOE_N_STAGES && !g_prof.has[c][j]) ++j;
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, g_prof.ev[c][i], g_prof.ev[c][j]) != hipSuccess)
                return GLMMOE_ERR_LAUNCH;
            stage_ms[i] += ms;
            n_calls[i] += 1;
        }
    }
    g_prof.calls = 0;
    return GLMMOE_OK;
}

}  // extern "C"
