/*
 * moe_oracle.h -- CPU restatement of glmserve's MoE-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP path in
 * glmserve_amd/: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product path never calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the glmserve source tree).
 *
 * Pinning status of each function (how a plausible mistake would be caught):
 *   orc_expf / orc_sigmoid  : vs libm exp/sigmoid over a dense sweep (<= 2 ulp)
 *                             and exact special values (tests/test_oracle.py).
 *   orc_bf16 conversions     : exhaustive over all 65536 bf16 patterns and RNE
 *                             tie cases (tests/test_oracle.py).
 *   orc_linear_f32           : bit-exact vs the compiled reference
 *                             linear_forward via oracle/_ref (the router logits
 *                             inside moe_mlp) and fp64 brute force.
 *   orc_router_logits_bf16   : exact on integer-valued inputs (order-free),
 *                             fp64 brute force within the fp32 error bound,
 *                             and bit-exact vs orc_linear_f32 when H <= 128.
 *   orc_router_topk          : brute-force full stable sort on many random
 *                             rows, forced ties, wsum == 0, norm off, and the
 *                             whole-layer comparison vs oracle/_ref.
 *   orc_dispatch             : brute-force stable sort + invariants.
 *   orc_dequant_int4_rows    : exhaustive nibble x scale, bit-exact vs the
 *                             reference dequant_int4_to_f32 in oracle/_ref.
 *   orc_moe_forward          : vs the compiled reference GLM52Model::moe_mlp
 *                             (oracle/_ref) on the tiny config, and vs an fp64
 *                             brute force; special cases k=1/w=1 (plain SwiGLU),
 *                             zero up-projection gives zero routed output.
 *   orc_e4m3 conversions     : exhaustive 256-entry decode and RNE encode vs
 *                             torch float8_e4m3fn (tests/test_oracle.py).
 *   orc_quant_act_e4m3       : vs torch's float8_e4m3fn conversion of x/scale,
 *                             scale = amax/448 closed form, |x - deq| bound.
 *   orc_dequant_e4m3_blocks  : closed form per element, block index mapping.
 *   orc_quant_act_q8         : numpy float32 closed form (sx = amax / 127,
 *                             RNE of v * (1 / sx)) and |x - sx * q| <= sx / 2.
 *   orc_gguf_frag_i8         : ds * wq - dm equals orc_gguf_value for every
 *                             element of random blocks of every int8 type.
 *   orc_gguf_*               : bit-exact vs the reference's gguf_dequantize_row
 *                             (oracle/_ref) on random blocks of every type,
 *                             codebooks byte-identical to the reference's,
 *                             and hand-built known-answer blocks.
 */
#ifndef GLMMOE_ORACLE_H
#define GLMMOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float orc_expf(float x);
float orc_sigmoid(float x);
float orc_silu(float x);
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_n(const float* src, uint16_t* dst, int64_t count);
void orc_bf16_to_f32_n(const uint16_t* src, float* dst, int64_t count);

float orc_e4m3_to_f32(uint8_t v);
uint8_t orc_f32_to_e4m3(float f);
void orc_quant_act_e4m3(const float* x, int64_t n, int64_t K, uint8_t* q, float* scale);
void orc_dequant_e4m3_blocks(const uint8_t* q, const float* scales, int64_t rows, int64_t K,
                             float* out);

void orc_linear_f32(const float* x, const float* w, int64_t n, int64_t in, int64_t out,
                    float* y);
void orc_router_logits_bf16(const uint16_t* x, const uint16_t* wr, int64_t n, int64_t H,
                            int64_t E, float* logits);
int orc_router_topk(const float* logits, const float* e_bias, int64_t n, int E, int topk,
                    int norm_topk, float routed_scale, int* topk_ids, float* topk_w);
int orc_dispatch(const int* topk_ids, int64_t n, int topk, int E, int* expert_offsets,
                 int* sorted_token_ids, int* sorted_row);
void orc_dequant_int4_rows(const uint8_t* q, const float* scales, int64_t rows, int64_t in,
                           int64_t group_size, float* out);
void orc_quantize_w4_rows(const float* w, int64_t rows, int64_t in, int64_t group_size,
                          uint8_t* q, float* scales);

/* One MoE layer (moe_mlp semantics) on fp32 (dequantized) weights.
 * gate[e]/up[e]: [I, H]; down[e]: [H, I]; a NULL expert pointer means "not
 * materialized" and is an error if routing selects it. logits may be given
 * (logits_in != NULL) or computed with orc_linear_f32 from router_w [E, H].
 * Returns 0, or -1 if routing selected a NULL expert. */
int orc_moe_forward(const float* x, int64_t n, int64_t H, int E, int topk, int64_t I,
                    int64_t S, const float* router_w, const float* logits_in,
                    const float* e_bias, const float* const* gate, const float* const* up,
                    const float* const* down, const float* sh_gate, const float* sh_up,
                    const float* sh_down, int norm_topk, float routed_scale, int nthreads,
                    float* out, int* ids_out, float* w_out);

/* Same, with h_fp8 != 0 quantizing the intermediate h per 128 features to
 * e4m3 (orc_quant_act_e4m3's rule) and dequantizing it before the down
 * projection, as the FP8 layer does. Pass x already quantized-dequantized. */
int orc_moe_forward_ex(const float* x, int64_t n, int64_t H, int E, int topk, int64_t I,
                       int64_t S, const float* router_w, const float* logits_in,
                       const float* e_bias, const float* const* gate, const float* const* up,
                       const float* const* down, const float* sh_gate, const float* sh_up,
                       const float* sh_down, int norm_topk, float routed_scale, int h_fp8,
                       int nthreads, float* out, int* ids_out, float* w_out);


/* GGUF block formats (src/gguf_quant.cpp:98-262): element p of one block, a
 * whole row of n elements (n a multiple of the block size; -1 otherwise), the
 * block geometry, and the two codebooks (for pinning against the reference's). */
/* Expert FFN of m rows at once (orc_ffn per row, bit for bit) and the
 * slot-order combine of per-slot rows plus the shared rows; together they
 * equal orc_moe_forward_ex for the same routing. */
void orc_expert_rows(const float* x, int64_t m, int64_t H, int64_t I, const float* gate,
                     const float* up, const float* down, int h_fp8, int nthreads, float* y);
void orc_combine_slots(const float* slot_rows, const float* topk_w, const float* shared_rows,
                       int64_t n, int topk, int64_t H, float* out);

int64_t orc_gguf_block_elems(uint32_t type);
int64_t orc_gguf_block_bytes(uint32_t type);
float orc_gguf_value(uint32_t type, const uint8_t* block, int p);
int orc_gguf_dequant_row(uint32_t type, const uint8_t* src, int64_t n, float* dst);
void orc_gguf_tables(const uint32_t** iq3xxs_grid, const int8_t** iq4nl_values);


/* GGUF int8-activation path (cuda/qgemm.cu:104-303, 556-587): the activation
 * quantizer, the integer fragment form of 8 weights (weight = ds * wq - dm),
 * and gemm_q_i8's products summed per fragment in fp64. */
void orc_quant_act_q8(const float* x, int64_t n, int64_t in, int8_t* xq, float* xs);
int orc_gguf_frag_i8(uint32_t type, const uint8_t* row, int64_t k, int8_t* wq, float* ds,
                     float* dm);
int orc_gemm_q_i8(uint32_t type, const int8_t* xq, const float* xs, const uint8_t* w, int64_t n,
                  int64_t in, int64_t out, int64_t row_bytes, double* y);

#ifdef __cplusplus
}
#endif
#endif
