// Internal launchers shared by the kernel files and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace glmmoe {

// Grouped rows per tile of the decode expert GEMMs (one 16-token MFMA block).
constexpr int kTileRows = 16;
// Grouped rows per tile of the large-group (prefill) expert GEMMs.
constexpr int kBigRows = 128;
// Grouped rows (n*topk + n) from which the layer uses the large-group kernels.
constexpr int kBigMinRows = 1024;

struct ExpertPtrs {
    const uint8_t* gate_q; const uint16_t* gate_s;
    const uint8_t* up_q; const uint16_t* up_s;
    const uint8_t* down_q; const uint16_t* down_s;
    const uint8_t* sh_gate_q; const uint16_t* sh_gate_s;
    const uint8_t* sh_up_q; const uint16_t* sh_up_s;
    const uint8_t* sh_down_q; const uint16_t* sh_down_s;
};

// FP8 experts: packed e4m3 tiles and fp32 128 x 128 block scales per matrix.
struct Fp8Ptrs {
    const uint8_t* gate_q; const float* gate_s;
    const uint8_t* up_q; const float* up_s;
    const uint8_t* down_q; const float* down_s;
    const uint8_t* sh_gate_q; const float* sh_gate_s;
    const uint8_t* sh_up_q; const float* sh_up_s;
    const uint8_t* sh_down_q; const float* sh_down_s;
};

// Outputs of a dispatch. mode bit 0: also emit inv[], the shared-expert rows
// and the tile list (layer path).
struct DispOut {
    int* offsets;
    int* sorted_tok;
    int* sorted_slot;
    int* inv;
    int4* tiles;
    int* ntiles;
    int tile_rows;
    int with_shared;
    int mode;
    int half_rows;   // > 0: tail tiles of at most this many rows listed last; < 0: ntiles has one int
    unsigned int* zero;   // nzero words the dispatch sets to 0 (the expert kernels' tickets), or null
    int nzero;
};

// Scratch (bytes) the router-logit launch needs for n tokens; 0 for large n.
size_t router_logits_scratch_bytes(int n, int H, int E);
int launch_router_logits(const uint16_t* x, const uint16_t* wr, int n, int H, int E,
                         float* logits, float* xsum, float* scratch, hipStream_t s);
// fp32 x [n, H] and W [E, H] rounded to bf16 on load, the bf16 path's fixed
// order, + bias (nullable). H % 128 == 0, H <= 8192; no workspace.
int launch_router_logits_f32(const float* x, const float* W, const float* bias, float* y, int n,
                             int H, int E, hipStream_t s);
int launch_xsum(const uint16_t* x, int n, int H, float* xsum, hipStream_t s);
// Router logits + top-k for the layer (logits hold only what the selection
// reads; ids and weights are those of the fixed-order logits). Scratch of
// router_select_scratch_bytes.
size_t router_select_scratch_bytes(int n, int H, int E);
int launch_router_select(const uint16_t* x, const uint16_t* wr, const float* e_bias, int n, int H,
                         int E, int topk, int norm_topk, float routed_scale, float* logits,
                         float* xsum, float* scratch, int* ids, float* w, hipStream_t s,
                         const DispOut* disp = nullptr, bool* dispatched = nullptr,
                         bool select = true, const float* xf = nullptr, uint16_t* xb = nullptr,
                         uint16_t* xh = nullptr, float* xrho = nullptr, bool* x16_done = nullptr);
// xh / xrho (nullable): where the large-group gate/up kernel reads x as fp16
// rows ([n, H]) and their factors ([n]); the router writes them (the
// conversion launch_gate_up_big otherwise runs) when it stages whole rows
// (from kTiledMinTokens tokens) and then sets *x16_done.
// xf (small-batch path only): fp32 activations [n, H], rounded to bf16 as the
// router stages them; the rounded rows are written to xb ([n, H]) and x is
// not read.
// The small-batch router path (router_small_kernel) applies to this shape.
// With select == false launch_router_select then only writes the logits, the
// order codes and scores ([2][n][E] in scratch) and xsum, and zeroes
// disp->zero (the tickets): the selection and dispatch run inside gate/up.
bool router_small_path(int n, int H, int E, int topk);
int launch_router_topk(const float* logits, const float* e_bias, int n, int E, int topk,
                       int norm_topk, float routed_scale, int* ids, float* w, hipStream_t s);
// Scratch (bytes) the multi-workgroup dispatch of a large batch uses (0 below it).
size_t dispatch_scratch_bytes(int n, int topk, int E);
int launch_dispatch(const int* ids, int n, int topk, int E, int* offsets, int* sorted_tok,
                    int* sorted_slot, int* inv, int* tiles, int* ntiles, int tile_rows,
                    int with_shared, int mode, hipStream_t s, int* scratch = nullptr,
                    int half_rows = -1, unsigned int* zero = nullptr, int nzero = 0);
int launch_pack_w4(const uint8_t* q, const void* sc, int sc_bf16, int n_mats, int rows, int K,
                   uint8_t* pq, uint16_t* ps, hipStream_t s);
// tick: kTailTicks words, zero at launch (the router or dispatch kernel clears them); tpart:
// tpart_bytes of scratch for split items' partials (no split without them).
constexpr int kTailTicks = 256;
// Selection and dispatch of a small batch (n <= kFusedRouteMax) inside the
// gate/up stream kernel: each workgroup selects the tokens' experts from
// router_small_kernel's order codes and scores (the router's top-k, one wave
// per token) and dispatches them into its LDS; workgroup 0 also stores the
// ids, weights and dispatch outputs the later kernels read.
constexpr int kFusedRouteMax = 8;
struct FusedRoute {
    const uint32_t* cs;   // order codes [n][E], then scores [n][E]
    int n, topk, norm_topk;
    float routed_scale;
    int* ids;             // [n][topk]
    float* w;
    DispOut disp;         // global outputs (tile_rows kTileRows, mode 1, half_rows 0)
};
// Whether gate/up can take the fused selection for this shape.
bool fused_route_ok(int n, int topk, int E, int H);
int launch_gate_up(const ExpertPtrs& P, const uint16_t* x, const float* xsum, const int* tiles,
                   const int* ntiles, int max_tiles, const int* rows_tok, uint16_t* h,
                   float* hsum, unsigned int* tick, float* tpart, size_t tpart_bytes, int H, int I,
                   int E, hipStream_t s, const FusedRoute* route = nullptr,
                   bool stream_weights = false);
// stream_weights: the decode kernels read the expert weights with
// non-temporal loads (a batch whose routed weights exceed the last-level
// cache: they are read once, and the activation rows stay in L2).
int launch_down(const ExpertPtrs& P, const uint16_t* h, const float* hsum, const int* tiles,
                const int* ntiles, int max_tiles, float* dpart, int H, int I, int E,
                hipStream_t s, bool stream_weights = false);
// Shapes the large-group W4A16 kernels take: H / 128 and I / 128 multiples of 8.
bool big_w4_shape_ok(int H, int I);
// Large-group kernels (fp16 MFMA). gate/up converts x to fp16 rows in scratch
// (at least n * H * 2 + n * 4 bytes, free until down) and writes h as fp16
// rows with a power-of-2 exponent per 32-feature block in hexp ([R, I / 32]
// bytes); down first brings each of the R rows to one exponent, then undoes it.
int launch_gate_up_big(const ExpertPtrs& P, const uint16_t* x, int n, const int* tiles,
                       const int* ntiles, int max_tiles, const int* rows_tok, uint16_t* h,
                       int8_t* hexp, void* scratch, size_t scratch_bytes, unsigned int* tick, int H,
                       int I, int E, hipStream_t s, bool x16_ready = false);
// log2 of the factor the large-group kernels' weight decode applies to the
// scales (and their epilogues undo).
constexpr int kWPre = 8;
int launch_down_big(const ExpertPtrs& P, uint16_t* h, int8_t* hexp, int R, const int* tiles,
                    const int* ntiles, int max_tiles, float* dpart, int H, int I, int E,
                    hipStream_t s);
// bf16: the partial rows are bf16 (written by the large-group kernels).
int launch_combine(const float* dpart, const int* inv, const float* w, int n, int topk, int H,
                   int with_shared, float* out, hipStream_t s, bool bf16 = false);

int launch_quant_act_fp8(const uint16_t* x, int n, int K, uint8_t* q, float* scale,
                         hipStream_t s);
int launch_pack_fp8(const uint8_t* w, int n_mats, int rows, int K, uint8_t* packed,
                    hipStream_t s);
int launch_gate_up_fp8(const Fp8Ptrs& P, const uint8_t* xq, const float* xscale,
                       const int* tiles, const int* ntiles, int max_tiles, const int* rows_tok,
                       uint8_t* hq, float* hscale, int H, int I, int E, hipStream_t s);
int launch_down_fp8(const Fp8Ptrs& P, const uint8_t* hq, const float* hscale, const int* tiles,
                    const int* ntiles, int max_tiles, float* dpart, int H, int I, int E,
                    hipStream_t s);


// Reference-signature kernels (compat.hip).
int launch_ref_gemm_w4(const float* x, const uint8_t* qw, const float* sc, const float* bias,
                       float* y, int n, int in, int out, int g, hipStream_t s);
int launch_ref_gemm_fp8(const float* x, const uint8_t* w, const float* sc, const float* bias,
                        float* y, int n, int in, int out, hipStream_t s);
int launch_ref_expert_f32(const float* x, const int* ids, const float* w, const float* gw,
                          const float* uw, const float* dw, int n, int topk, int H, int I,
                          float* out, hipStream_t s);
int launch_ref_silu_mul(const float* g, const float* u, float* o, long n, hipStream_t s);
int launch_ref_add_inplace(float* y, const float* x, long n, hipStream_t s);
int launch_f32_to_bf16(const float* x, uint16_t* y, long n, hipStream_t s);

// GGUF block formats (gguf.hip): block geometry (0 if unsupported) and the
// gemm_q / moe_expert_ffn_q launches.
int gguf_block_elems(uint32_t type);
int gguf_block_bytes(uint32_t type);
int launch_gg_gemm(uint32_t qtype, const float* x, const uint8_t* qw, const float* bias, float* y,
                   int n, int in, int out, long row_bytes, hipStream_t s);
int launch_gg_moe(uint32_t gt, uint32_t ut, uint32_t dt, const float* x, const int* ids,
                  const float* w, const uint8_t* gq, const uint8_t* uq, const uint8_t* dq, int n,
                  int topk, int H, int I, int E, long grb, long urb, long drb, float* h_act,
                  float* dpart, float* out, int* dispatch, hipStream_t s);
// int8-activation twins (quantize_act_q8, gemm_q_i8, moe_expert_ffn_q_i8).
bool gguf_has_i8(uint32_t type);
int launch_gg_quant_q8(const float* x, long total, int8_t* xq, float* xs, hipStream_t s);
int launch_gg_gemm_i8(uint32_t qtype, const int8_t* xq, const float* xs, const uint8_t* qw,
                      const float* bias, float* y, int n, int in, int out, long row_bytes,
                      hipStream_t s);
int launch_gg_moe_i8(uint32_t gt, uint32_t ut, uint32_t dt, const int8_t* xq, const float* xs,
                     const int* ids, const float* w, const uint8_t* gq, const uint8_t* uq,
                     const uint8_t* dq, int n, int topk, int H, int I, int E, long grb, long urb,
                     long drb, float* h_act, int8_t* hq, float* hs, float* dpart, float* out,
                     int* dispatch, hipStream_t s);

}  // namespace glmmoe
