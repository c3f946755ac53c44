/*
 * moe_oracle.c -- CPU restatement of glmserve's MoE-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never part of
 * the product path. Built with -ffp-contract=off so that every floating-point
 * operation rounds exactly where it is written (fmaf() is called explicitly
 * where a fused multiply-add is meant).
 *
 * Reference citations are paths in the glmserve tree.
 */
#include "moe_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------
 * exp / sigmoid / silu.
 * The reference uses std::exp on the CPU (src/model_glm52.cpp:95-96) and the
 * __expf intrinsic on the GPU (cuda/common.cuh:53-54); the two disagree in the
 * last bits. This build defines ONE exp that the CPU oracle and the HIP
 * kernels both evaluate operation-for-operation, so sigmoid scores (and thus
 * routing) are bit-identical across the two:
 *   Cody-Waite range reduction x = n*ln2 + r, |r| <= ln2/2, with ln2 split into
 *   a 24-bit-exact high part and a low correction (Cody & Waite, "Software
 *   Manual for the Elementary Functions", 1980), then the degree-7 Taylor
 *   polynomial of e^r in Horner form (truncation error < 6e-9 relative on
 *   |r| <= 0.347), then scaling by 2^n built from exponent bits.
 * The argument is clamped to [-80, 80] so 2^n is always a normal float and no
 * denormal handling differs between CPU and GPU. sigmoid(x) for |x| > 80 is
 * therefore computed at +-80 (it differs from the true value only below
 * 2e-35, or by less than 2^-24 from 1).
 * ------------------------------------------------------------------------- */
#define ORC_LOG2E 1.44269504088896341f
#define ORC_LN2_HI 0.693145751953125f      /* 0x3f317200, exact in 16 bits */
#define ORC_LN2_LO 1.42860682030941723e-06f /* ln2 - LN2_HI */

float orc_expf(float x) {
    if (x != x) return x;
    if (x > 80.0f) x = 80.0f;
    if (x < -80.0f) x = -80.0f;
    float n = rintf(x * ORC_LOG2E);
    float r = fmaf(-n, ORC_LN2_HI, x);
    r = fmaf(-n, ORC_LN2_LO, r);
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ni = (int)n;
    uint32_t bits = (uint32_t)(ni + 127) << 23;
    float scale;
    memcpy(&scale, &bits, sizeof scale);
    return p * scale;
}

/* sigmoidf: src/model_glm52.cpp:96 (1 / (1 + exp(-x))). */
float orc_sigmoid(float x) { return 1.0f / (1.0f + orc_expf(-x)); }

/* silu: src/model_glm52.cpp:95 (x / (1 + exp(-x))). */
float orc_silu(float x) { return x / (1.0f + orc_expf(-x)); }

/* bf16 <-> f32: include/common.hpp:121-136 (top 16 bits; RNE on the way down).
 * NaN inputs are kept NaN (quiet bit forced), which the reference's add-bias
 * trick does not guarantee; finite and infinite values match it exactly. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, sizeof bits);
    if ((bits & 0x7f800000u) == 0x7f800000u && (bits & 0x007fffffu))
        return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t lsb = (bits >> 16) & 1u;
    bits += 0x7fffu + lsb;
    return (uint16_t)(bits >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

void orc_f32_to_bf16_n(const float* src, uint16_t* dst, int64_t count) {
    for (int64_t i = 0; i < count; ++i) dst[i] = orc_f32_to_bf16(src[i]);
}

void orc_bf16_to_f32_n(const uint16_t* src, float* dst, int64_t count) {
    for (int64_t i = 0; i < count; ++i) dst[i] = orc_bf16_to_f32(src[i]);
}

/* FP8 e4m3 decode: include/common.hpp:182-200 (bias 7, no infinities; the
 * reference decodes 0x7f/0xff as +-480 rather than NaN -- restated as is; the
 * encoder below never produces those two codes). */
float orc_e4m3_to_f32(uint8_t v) {
    float sign = (v & 0x80u) ? -1.0f : 1.0f;
    int e = (v >> 3) & 0xf;
    int m = v & 0x7;
    if (e == 0) return sign * ldexpf((float)m, -9);
    return sign * ldexpf(1.0f + (float)m / 8.0f, e - 7);
}

/* FP8 e4m3 encode, round-to-nearest-even, saturating to +-448 (the largest
 * OCP e4m3fn finite value), so the NaN codes never appear. No reference
 * counterpart (the reference only decodes FP8, src/tensor.cpp:21-24). */
uint8_t orc_f32_to_e4m3(float f) {
    uint8_t s = signbit(f) ? 0x80u : 0u;
    float a = fabsf(f);
    if (a != a) return (uint8_t)(s | 0x7e);
    if (a >= 448.0f) return (uint8_t)(s | 0x7e);
    if (a < 0.015625f) { /* subnormal range, step 2^-9 */
        int m = (int)rintf(a * 512.0f);
        return (uint8_t)(s | m); /* m == 8 is exactly the min normal code 0x08 */
    }
    int ex;
    float fr = frexpf(a, &ex); /* a = fr * 2^ex, fr in [0.5, 1) */
    int e = ex - 1;
    int m = (int)rintf((fr * 2.0f - 1.0f) * 8.0f);
    if (m == 8) { m = 0; ++e; }
    return (uint8_t)(s | ((e + 7) << 3) | m);
}

/* Per-token, per-128-channel FP8 quantization of activations (the FP8
 * workload of this build's benchmark; the reference has no FP8 MoE, its FP8
 * code only decodes weights, cuda/fp8_gemm.cu:14-35). For every row and every
 * group of 128 columns: amax = max |x|, scale = amax / 448 (1 when amax is
 * 0), q = e4m3(x / scale) with round-to-nearest-even and saturation. */
void orc_quant_act_e4m3(const float* x, int64_t n, int64_t K, uint8_t* q, float* scale) {
    int64_t G = K / 128;
    for (int64_t t = 0; t < n; ++t)
        for (int64_t g = 0; g < G; ++g) {
            const float* xs = x + t * K + g * 128;
            float amax = 0.0f;
            for (int i = 0; i < 128; ++i) {
                float a = fabsf(xs[i]);
                if (a > amax) amax = a;
            }
            float s = amax > 0.0f ? amax / 448.0f : 1.0f;
            scale[t * G + g] = s;
            for (int i = 0; i < 128; ++i) q[t * K + g * 128 + i] = orc_f32_to_e4m3(xs[i] / s);
        }
}

/* FP8 weight [rows, K] (row-major e4m3 bytes) with fp32 scales per 128 x 128
 * block [rows/128, K/128] -> fp32 (w = e4m3(q) * block scale). */
void orc_dequant_e4m3_blocks(const uint8_t* q, const float* scales, int64_t rows, int64_t K,
                             float* out) {
    int64_t KB = K / 128;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t k = 0; k < K; ++k)
            out[r * K + k] = orc_e4m3_to_f32(q[r * K + k]) * scales[(r / 128) * KB + k / 128];
}

/* linear_forward: src/model_glm52.cpp:42-56. y[n,out] = x[n,in] . W[out,in]^T,
 * one scalar fp32 accumulator per output, ascending i, acc += x*w with the
 * product rounded before the add (the reference is built -std=c++17 -O2 for
 * x86-64 without FMA, so no contraction). */
void orc_linear_f32(const float* x, const float* w, int64_t n, int64_t in, int64_t out,
                    float* y) {
    for (int64_t t = 0; t < n; ++t) {
        const float* xt = x + t * in;
        for (int64_t o = 0; o < out; ++o) {
            const float* wo = w + o * in;
            float acc = 0.0f;
            for (int64_t i = 0; i < in; ++i) {
                float p = xt[i] * wo[i];
                acc = acc + p;
            }
            y[t * out + o] = acc;
        }
    }
}

/* Router logits with bf16 inputs in this build's fixed reduction order (the
 * reference's GPU path goes through cublasSgemm, cuda/gemm.cu:62-78, whose
 * order is unspecified; its CPU path is linear_forward above):
 *   K is cut into chunks of 128; each chunk is summed from zero in ascending
 *   order, and the chunk sums are added to the total in ascending chunk order.
 * bf16 x bf16 products are exact in fp32, so fmaf(x, w, s) == s + x*w and the
 * per-chunk sum is exactly linear_forward's order restarted every 128 inputs.
 * For H <= 128 this IS linear_forward. */
#define ORC_ROUTER_KC 128
void orc_router_logits_bf16(const uint16_t* x, const uint16_t* wr, int64_t n, int64_t H,
                            int64_t E, float* logits) {
    for (int64_t t = 0; t < n; ++t) {
        const uint16_t* xt = x + t * H;
        for (int64_t e = 0; e < E; ++e) {
            const uint16_t* we = wr + e * H;
            float total = 0.0f;
            for (int64_t c = 0; c < H; c += ORC_ROUTER_KC) {
                int64_t ce = c + ORC_ROUTER_KC < H ? c + ORC_ROUTER_KC : H;
                float s = 0.0f;
                for (int64_t i = c; i < ce; ++i)
                    s = fmaf(orc_bf16_to_f32(xt[i]), orc_bf16_to_f32(we[i]), s);
                total = total + s;
            }
            logits[t * E + e] = total;
        }
    }
}

/* Routing: the GPU kernel cuda/moe_router.cu:17-72 and the CPU loop
 * src/model_glm52.cpp:1113-1129.
 *   score = sigmoid(logit); choose = score + e_bias (e_bias may be NULL);
 *   k rounds: pick the not-yet-taken expert with the largest choose, ties to
 *   the lower expert index (moe_router.cu:48-53); NaN never wins;
 *   weight = the UNBIASED score, wsum accumulated in selection order;
 *   if norm_topk and wsum > 0: w /= wsum; then w *= routed_scale.
 * Returns 0, or -1 on a bad shape (E < topk, topk < 1). */
int orc_router_topk(const float* logits, const float* e_bias, int64_t n, int E, int topk,
                    int norm_topk, float routed_scale, int* topk_ids, float* topk_w) {
    if (topk < 1 || E < topk) return -1;
    float* score = (float*)malloc(sizeof(float) * (size_t)E);
    float* choose = (float*)malloc(sizeof(float) * (size_t)E);
    unsigned char* taken = (unsigned char*)malloc((size_t)E);
    for (int64_t t = 0; t < n; ++t) {
        const float* lt = logits + t * E;
        for (int e = 0; e < E; ++e) {
            score[e] = orc_sigmoid(lt[e]);
            choose[e] = score[e] + (e_bias ? e_bias[e] : 0.0f);
            taken[e] = 0;
        }
        int* ids = topk_ids + t * topk;
        float* w = topk_w + t * topk;
        float wsum = 0.0f;
        for (int k = 0; k < topk; ++k) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                if (taken[e]) continue;
                if (best < 0) { best = e; continue; }
                float c = choose[e], b = choose[best];
                if (b != b) { if (c == c) best = e; continue; }   /* NaN loses */
                if (c > b) best = e;                               /* strict: ties keep lower */
            }
            taken[best] = 1;
            ids[k] = best;
            w[k] = score[best];
            wsum = wsum + score[best];
        }
        for (int k = 0; k < topk; ++k) {
            float v = w[k];
            if (norm_topk && wsum > 0.0f) v = v / wsum;
            w[k] = v * routed_scale;
        }
    }
    free(score);
    free(choose);
    free(taken);
    return 0;
}

/* Dispatch: cuda/moe_dispatch.cu:16-39 -- a counting sort over experts that
 * is stable in (token ascending, slot ascending) order within each expert.
 * expert_offsets[E+1] is the exclusive prefix of the per-expert counts;
 * sorted_row holds the slot k of each grouped row. Returns -1 on an
 * out-of-range id. */
int orc_dispatch(const int* topk_ids, int64_t n, int topk, int E, int* expert_offsets,
                 int* sorted_token_ids, int* sorted_row) {
    int64_t total = n * topk;
    for (int e = 0; e <= E; ++e) expert_offsets[e] = 0;
    for (int64_t i = 0; i < total; ++i) {
        int e = topk_ids[i];
        if (e < 0 || e >= E) return -1;
        expert_offsets[e + 1]++;
    }
    for (int e = 0; e < E; ++e) expert_offsets[e + 1] += expert_offsets[e];
    int* cursor = (int*)malloc(sizeof(int) * (size_t)(E > 0 ? E : 1));
    for (int e = 0; e < E; ++e) cursor[e] = expert_offsets[e];
    for (int64_t t = 0; t < n; ++t)
        for (int k = 0; k < topk; ++k) {
            int e = topk_ids[t * topk + k];
            int dst = cursor[e]++;
            sorted_token_ids[dst] = (int)t;
            sorted_row[dst] = k;
        }
    free(cursor);
    return 0;
}

/* int4 dequant of a [rows, in] matrix stored as packed [rows, ceil(in/2)] plus
 * scales [rows, ceil(in/g)]: src/tensor.cpp:53-63 per row (low nibble = even
 * column, value = (nibble - 8) * scale), the row layout of
 * cuda/moe_expert.cu:132-140. */
void orc_dequant_int4_rows(const uint8_t* q, const float* scales, int64_t rows, int64_t in,
                           int64_t group_size, float* out) {
    int64_t packed_in = (in + 1) / 2, groups = (in + group_size - 1) / group_size;
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t* qr = q + r * packed_in;
        const float* sr = scales + r * groups;
        for (int64_t i = 0; i < in; ++i) {
            uint8_t b = qr[i >> 1];
            int v = (i & 1) ? (b >> 4) : (b & 0x0f);
            out[r * in + i] = (float)(v - 8) * sr[i / group_size];
        }
    }
}

/* Symmetric int4 quantizer: tools/convert_hf_to_glmserve.py:216-252
 * (scale = max|x_g| / 7, 1.0 when the group is all zero; q = clip(rint(x/s),
 * -8, 7) + 8; low nibble = even column). */
void orc_quantize_w4_rows(const float* w, int64_t rows, int64_t in, int64_t group_size,
                          uint8_t* q, float* scales) {
    int64_t packed_in = (in + 1) / 2, groups = (in + group_size - 1) / group_size;
    memset(q, 0, (size_t)(rows * packed_in));
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t g = 0; g < groups; ++g) {
            int64_t c0 = g * group_size, c1 = c0 + group_size < in ? c0 + group_size : in;
            float amax = 0.0f;
            for (int64_t i = c0; i < c1; ++i) {
                float a = fabsf(w[r * in + i]);
                if (a > amax) amax = a;
            }
            float s = amax / 7.0f;
            if (!(s > 0.0f)) s = 1.0f;
            scales[r * groups + g] = s;
            for (int64_t i = c0; i < c1; ++i) {
                float v = rintf(w[r * in + i] / s);
                if (v < -8.0f) v = -8.0f;
                if (v > 7.0f) v = 7.0f;
                int qi = (int)v + 8;
                q[r * packed_in + (i >> 1)] |= (uint8_t)((i & 1) ? (qi << 4) : qi);
            }
        }
    }
}

/* ---------------------------------------------------------------------------
 * Whole layer: GLM52Model::moe_mlp, src/model_glm52.cpp:1096-1154.
 * Per token: route (above), then for each slot kk in selection order
 *   g = gate.x, u = up.x (linear_forward), h = silu(g)*u, tmp = down.h,
 *   out += w[kk]*tmp; then the shared expert adds with weight 1.
 * out starts at zero (:1107).
 * ------------------------------------------------------------------------- */
typedef struct {
    const float* x;
    int64_t n, H, I, S;
    int E, topk;
    const float* logits;
    const float* e_bias;
    const float* const* gate;
    const float* const* up;
    const float* const* down;
    const float *sh_gate, *sh_up, *sh_down;
    int norm_topk;
    float routed_scale;
    float* out;
    int* ids;
    float* w;
    int64_t t0, t1;
    int h_fp8;
    int status;
} orc_job;

/* h_fp8: the FP8 layer's intermediate, h quantized per 128 features with
 * orc_quant_act_e4m3's rule and dequantized (e4m3(q) * scale) before the down
 * projection. */
static void orc_ffn(const float* xt, const float* g_w, const float* u_w, const float* d_w,
                    int64_t H, int64_t I, int h_fp8, float* g, float* u, float* tmp) {
    orc_linear_f32(xt, g_w, 1, H, I, g);
    orc_linear_f32(xt, u_w, 1, H, I, u);
    for (int64_t i = 0; i < I; ++i) g[i] = orc_silu(g[i]) * u[i];
    if (h_fp8) {
        for (int64_t g0 = 0; g0 < I; g0 += 128) {
            uint8_t q[128];
            float sc;
            orc_quant_act_e4m3(g + g0, 1, 128, q, &sc);
            for (int i = 0; i < 128; ++i) g[g0 + i] = orc_e4m3_to_f32(q[i]) * sc;
        }
    }
    orc_linear_f32(g, d_w, 1, I, H, tmp);
}

static void* orc_moe_worker(void* arg) {
    orc_job* j = (orc_job*)arg;
    int64_t I = j->I > j->S ? j->I : j->S;
    float* g = (float*)malloc(sizeof(float) * (size_t)I);
    float* u = (float*)malloc(sizeof(float) * (size_t)I);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)j->H);
    for (int64_t t = j->t0; t < j->t1; ++t) {
        const float* xt = j->x + t * j->H;
        int* ids = j->ids + t * j->topk;
        float* w = j->w + t * j->topk;
        orc_router_topk(j->logits + t * j->E, j->e_bias, 1, j->E, j->topk, j->norm_topk,
                        j->routed_scale, ids, w);
        float* ot = j->out + t * j->H;
        for (int64_t i = 0; i < j->H; ++i) ot[i] = 0.0f;
        for (int kk = 0; kk < j->topk; ++kk) {
            int e = ids[kk];
            if (!j->gate[e] || !j->up[e] || !j->down[e]) { j->status = -1; continue; }
            orc_ffn(xt, j->gate[e], j->up[e], j->down[e], j->H, j->I, j->h_fp8, g, u, tmp);
            for (int64_t i = 0; i < j->H; ++i) ot[i] = ot[i] + w[kk] * tmp[i];
        }
        if (j->sh_gate) {
            orc_ffn(xt, j->sh_gate, j->sh_up, j->sh_down, j->H, j->S, j->h_fp8, g, u, tmp);
            for (int64_t i = 0; i < j->H; ++i) ot[i] = ot[i] + tmp[i];
        }
    }
    free(g);
    free(u);
    free(tmp);
    return NULL;
}

int orc_moe_forward(const float* x, int64_t n, int64_t H, int E, int topk, int64_t I,
                    int64_t S, const float* router_w, const float* logits_in,
                    const float* e_bias, const float* const* gate, const float* const* up,
                    const float* const* down, const float* sh_gate, const float* sh_up,
                    const float* sh_down, int norm_topk, float routed_scale, int nthreads,
                    float* out, int* ids_out, float* w_out) {
    return orc_moe_forward_ex(x, n, H, E, topk, I, S, router_w, logits_in, e_bias, gate, up,
                              down, sh_gate, sh_up, sh_down, norm_topk, routed_scale, 0,
                              nthreads, out, ids_out, w_out);
}

int orc_moe_forward_ex(const float* x, int64_t n, int64_t H, int E, int topk, int64_t I,
                       int64_t S, const float* router_w, const float* logits_in,
                       const float* e_bias, const float* const* gate, const float* const* up,
                       const float* const* down, const float* sh_gate, const float* sh_up,
                       const float* sh_down, int norm_topk, float routed_scale, int h_fp8,
                       int nthreads, float* out, int* ids_out, float* w_out) {
    float* logits = NULL;
    const float* lg = logits_in;
    if (!lg) {
        logits = (float*)malloc(sizeof(float) * (size_t)(n * E));
        orc_linear_f32(x, router_w, n, H, E, logits);
        lg = logits;
    }
    if (nthreads < 1) nthreads = 1;
    if (nthreads > n) nthreads = (int)(n > 0 ? n : 1);
    orc_job* jobs = (orc_job*)calloc((size_t)nthreads, sizeof(orc_job));
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    int64_t chunk = (n + nthreads - 1) / nthreads;
    for (int i = 0; i < nthreads; ++i) {
        orc_job* j = &jobs[i];
        j->x = x; j->n = n; j->H = H; j->I = I; j->S = S; j->E = E; j->topk = topk;
        j->logits = lg; j->e_bias = e_bias; j->gate = gate; j->up = up; j->down = down;
        j->sh_gate = sh_gate; j->sh_up = sh_up; j->sh_down = sh_down;
        j->norm_topk = norm_topk; j->routed_scale = routed_scale;
        j->out = out; j->ids = ids_out; j->w = w_out; j->h_fp8 = h_fp8;
        j->t0 = i * chunk; j->t1 = (i + 1) * chunk < n ? (i + 1) * chunk : n;
        if (j->t0 > j->t1) j->t0 = j->t1;
    }
    if (nthreads == 1) {
        orc_moe_worker(&jobs[0]);
    } else {
        for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, orc_moe_worker, &jobs[i]);
        for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
    }
    int status = 0;
    for (int i = 0; i < nthreads; ++i) if (jobs[i].status) status = jobs[i].status;
    free(jobs);
    free(th);
    free(logits);
    return status;
}

/* ---------------------------------------------------------------------------
 * The layer streamed expert by expert, for full-output checks at large n.
 * orc_expert_rows runs orc_ffn's arithmetic on m rows of one expert at once:
 * every output element is the same scalar fp32 chain as orc_linear_f32
 * (ascending i, product rounded before the add), so each row equals orc_ffn on
 * that row bit for bit. Rows are processed in blocks of ORC_RB, transposed so
 * that the ORC_RB independent chains of one output sit side by side in memory
 * (the compiler can keep them in vector registers without reassociating any
 * chain). orc_combine_slots then adds the per-slot rows in slot order and the
 * shared row last, exactly as orc_moe_worker does (src/model_glm52.cpp:1133-1152):
 *   out[t] = ((0 + w0*y0) + w1*y1 + ...) + y_shared.
 * ------------------------------------------------------------------------- */
#define ORC_RB 32
__attribute__((optimize("O3"))) static void orc_linear_block(const float* xT, int64_t in, const float* w, int64_t out,
                             float* yT /* [out][ORC_RB] */) {
    for (int64_t o = 0; o < out; ++o) {
        const float* wo = w + o * in;
        float acc[ORC_RB];
        for (int r = 0; r < ORC_RB; ++r) acc[r] = 0.0f;
        for (int64_t i = 0; i < in; ++i) {
            const float wi = wo[i];
            const float* xi = xT + i * ORC_RB;
            for (int r = 0; r < ORC_RB; ++r) {
                float p = xi[r] * wi;
                acc[r] = acc[r] + p;
            }
        }
        for (int r = 0; r < ORC_RB; ++r) yT[o * ORC_RB + r] = acc[r];
    }
}

typedef struct {
    const float *x, *g_w, *u_w, *d_w;
    int64_t m, H, I;
    int h_fp8;
    float* y;
    int64_t b0, b1; /* row blocks of this worker */
} orc_rows_job;

static void* orc_rows_worker(void* arg) {
    orc_rows_job* j = (orc_rows_job*)arg;
    const int64_t H = j->H, I = j->I;
    float* xT = (float*)malloc(sizeof(float) * (size_t)(H * ORC_RB));
    float* gT = (float*)malloc(sizeof(float) * (size_t)(I * ORC_RB));
    float* uT = (float*)malloc(sizeof(float) * (size_t)(I * ORC_RB));
    float* yT = (float*)malloc(sizeof(float) * (size_t)(H * ORC_RB));
    for (int64_t b = j->b0; b < j->b1; ++b) {
        const int64_t r0 = b * ORC_RB;
        const int nr = (int)(j->m - r0 < ORC_RB ? j->m - r0 : ORC_RB);
        for (int64_t i = 0; i < H; ++i)
            for (int r = 0; r < ORC_RB; ++r)
                xT[i * ORC_RB + r] = r < nr ? j->x[(r0 + r) * H + i] : 0.0f;
        orc_linear_block(xT, H, j->g_w, I, gT);
        orc_linear_block(xT, H, j->u_w, I, uT);
        for (int64_t i = 0; i < I * ORC_RB; ++i) gT[i] = orc_silu(gT[i]) * uT[i];
        if (j->h_fp8) {
            /* per row: quantize h per 128 features (orc_ffn's h_fp8 step) */
            for (int r = 0; r < nr; ++r)
                for (int64_t g0 = 0; g0 < I; g0 += 128) {
                    float hv[128];
                    uint8_t q[128];
                    float sc;
                    for (int i = 0; i < 128; ++i) hv[i] = gT[(g0 + i) * ORC_RB + r];
                    orc_quant_act_e4m3(hv, 1, 128, q, &sc);
                    for (int i = 0; i < 128; ++i) gT[(g0 + i) * ORC_RB + r] = orc_e4m3_to_f32(q[i]) * sc;
                }
        }
        orc_linear_block(gT, I, j->d_w, H, yT);
        for (int r = 0; r < nr; ++r)
            for (int64_t i = 0; i < H; ++i) j->y[(r0 + r) * H + i] = yT[i * ORC_RB + r];
    }
    free(xT);
    free(gT);
    free(uT);
    free(yT);
    return NULL;
}

void orc_expert_rows(const float* x, int64_t m, int64_t H, int64_t I, const float* gate,
                     const float* up, const float* down, int h_fp8, int nthreads, float* y) {
    const int64_t nb = (m + ORC_RB - 1) / ORC_RB;
    if (nb == 0) return;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > nb) nthreads = (int)nb;
    orc_rows_job* jobs = (orc_rows_job*)calloc((size_t)nthreads, sizeof(orc_rows_job));
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    for (int i = 0; i < nthreads; ++i) {
        orc_rows_job* j = &jobs[i];
        j->x = x; j->g_w = gate; j->u_w = up; j->d_w = down;
        j->m = m; j->H = H; j->I = I; j->h_fp8 = h_fp8; j->y = y;
        j->b0 = nb * i / nthreads;
        j->b1 = nb * (i + 1) / nthreads;
    }
    if (nthreads == 1) {
        orc_rows_worker(&jobs[0]);
    } else {
        for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, orc_rows_worker, &jobs[i]);
        for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
    }
    free(jobs);
    free(th);
}

void orc_combine_slots(const float* slot_rows /* [n*topk, H], row t*topk+kk */,
                       const float* topk_w, const float* shared_rows /* [n, H] or NULL */,
                       int64_t n, int topk, int64_t H, float* out) {
    for (int64_t t = 0; t < n; ++t) {
        float* ot = out + t * H;
        for (int64_t i = 0; i < H; ++i) ot[i] = 0.0f;
        for (int kk = 0; kk < topk; ++kk) {
            const float w = topk_w[t * topk + kk];
            const float* y = slot_rows + (t * topk + kk) * H;
            for (int64_t i = 0; i < H; ++i) ot[i] = ot[i] + w * y[i];
        }
        if (shared_rows)
            for (int64_t i = 0; i < H; ++i) ot[i] = ot[i] + shared_rows[t * H + i];
    }
}

/* ---------------------------------------------------------------------------
 * GGUF block formats (src/gguf_quant.cpp:98-262, the reference's CPU
 * dequantizers of the ggml block layouts; types 0 F32, 1 F16, 8 Q8_0, 11 Q3_K,
 * 12 Q4_K, 13 Q5_K, 14 Q6_K, 18 IQ3_XXS, 23 IQ4_XS). Restated per element:
 * orc_gguf_value(type, block, p) decodes element p of one block with the same
 * float operations, in the same order, as the reference's block loops, so
 * rows dequantize bit-identically (pinned against oracle/_ref).
 * The two codebooks are format data and must hold exactly ggml's values: the
 * IQ3_XXS grid (256 entries of 4 magnitudes) and the IQ4_NL values; the
 * IQ2 sign table is the 7-bit index with an even-parity eighth bit.
 * ------------------------------------------------------------------------- */
static const uint32_t orc_iq3xxs_grid[256] = {
    0x04040404u, 0x04040414u, 0x04040424u, 0x04040c0cu, 0x04040c1cu, 0x04040c3eu, 0x04041404u, 0x04041414u,
    0x04041c0cu, 0x04042414u, 0x04043e1cu, 0x04043e2cu, 0x040c040cu, 0x040c041cu, 0x040c0c04u, 0x040c0c14u,
    0x040c140cu, 0x040c142cu, 0x040c1c04u, 0x040c1c14u, 0x040c240cu, 0x040c2c24u, 0x040c3e04u, 0x04140404u,
    0x04140414u, 0x04140424u, 0x04140c0cu, 0x04141404u, 0x04141414u, 0x04141c0cu, 0x04141c1cu, 0x04141c3eu,
    0x04142c0cu, 0x04142c3eu, 0x04143e2cu, 0x041c040cu, 0x041c043eu, 0x041c0c04u, 0x041c0c14u, 0x041c142cu,
    0x041c3e04u, 0x04240c1cu, 0x04241c3eu, 0x04242424u, 0x04242c3eu, 0x04243e1cu, 0x04243e2cu, 0x042c040cu,
    0x042c043eu, 0x042c1c14u, 0x042c2c14u, 0x04341c2cu, 0x04343424u, 0x043e0c04u, 0x043e0c24u, 0x043e0c34u,
    0x043e241cu, 0x043e340cu, 0x0c04040cu, 0x0c04041cu, 0x0c040c04u, 0x0c040c14u, 0x0c04140cu, 0x0c04141cu,
    0x0c041c04u, 0x0c041c14u, 0x0c041c24u, 0x0c04243eu, 0x0c042c04u, 0x0c0c0404u, 0x0c0c0414u, 0x0c0c0c0cu,
    0x0c0c1404u, 0x0c0c1414u, 0x0c14040cu, 0x0c14041cu, 0x0c140c04u, 0x0c140c14u, 0x0c14140cu, 0x0c141c04u,
    0x0c143e14u, 0x0c1c0404u, 0x0c1c0414u, 0x0c1c1404u, 0x0c1c1c0cu, 0x0c1c2434u, 0x0c1c3434u, 0x0c24040cu,
    0x0c24042cu, 0x0c242c04u, 0x0c2c1404u, 0x0c2c1424u, 0x0c2c2434u, 0x0c2c3e0cu, 0x0c34042cu, 0x0c3e1414u,
    0x0c3e2404u, 0x14040404u, 0x14040414u, 0x14040c0cu, 0x14040c1cu, 0x14041404u, 0x14041414u, 0x14041434u,
    0x14041c0cu, 0x14042414u, 0x140c040cu, 0x140c041cu, 0x140c042cu, 0x140c0c04u, 0x140c0c14u, 0x140c140cu,
    0x140c1c04u, 0x140c341cu, 0x140c343eu, 0x140c3e04u, 0x14140404u, 0x14140414u, 0x14140c0cu, 0x14140c3eu,
    0x14141404u, 0x14141414u, 0x14141c3eu, 0x14142404u, 0x14142c2cu, 0x141c040cu, 0x141c0c04u, 0x141c0c24u,
    0x141c3e04u, 0x141c3e24u, 0x14241c2cu, 0x14242c1cu, 0x142c041cu, 0x142c143eu, 0x142c240cu, 0x142c3e24u,
    0x143e040cu, 0x143e041cu, 0x143e0c34u, 0x143e242cu, 0x1c04040cu, 0x1c040c04u, 0x1c040c14u, 0x1c04140cu,
    0x1c04141cu, 0x1c042c04u, 0x1c04342cu, 0x1c043e14u, 0x1c0c0404u, 0x1c0c0414u, 0x1c0c1404u, 0x1c0c1c0cu,
    0x1c0c2424u, 0x1c0c2434u, 0x1c14040cu, 0x1c14041cu, 0x1c140c04u, 0x1c14142cu, 0x1c142c14u, 0x1c143e14u,
    0x1c1c0c0cu, 0x1c1c1c1cu, 0x1c241c04u, 0x1c24243eu, 0x1c243e14u, 0x1c2c0404u, 0x1c2c0434u, 0x1c2c1414u,
    0x1c2c2c2cu, 0x1c340c24u, 0x1c341c34u, 0x1c34341cu, 0x1c3e1c1cu, 0x1c3e3404u, 0x24040424u, 0x24040c3eu,
    0x24041c2cu, 0x24041c3eu, 0x24042c1cu, 0x24042c3eu, 0x240c3e24u, 0x24141404u, 0x24141c3eu, 0x24142404u,
    0x24143404u, 0x24143434u, 0x241c043eu, 0x241c242cu, 0x24240424u, 0x24242c0cu, 0x24243424u, 0x242c142cu,
    0x242c241cu, 0x242c3e04u, 0x243e042cu, 0x243e0c04u, 0x243e0c14u, 0x243e1c04u, 0x2c040c14u, 0x2c04240cu,
    0x2c043e04u, 0x2c0c0404u, 0x2c0c0434u, 0x2c0c1434u, 0x2c0c2c2cu, 0x2c140c24u, 0x2c141c14u, 0x2c143e14u,
    0x2c1c0414u, 0x2c1c2c1cu, 0x2c240c04u, 0x2c24141cu, 0x2c24143eu, 0x2c243e14u, 0x2c2c0414u, 0x2c2c1c0cu,
    0x2c342c04u, 0x2c3e1424u, 0x2c3e2414u, 0x34041424u, 0x34042424u, 0x34042434u, 0x34043424u, 0x340c140cu,
    0x340c340cu, 0x34140c3eu, 0x34143424u, 0x341c1c04u, 0x341c1c34u, 0x34242424u, 0x342c042cu, 0x342c2c14u,
    0x34341c1cu, 0x343e041cu, 0x343e140cu, 0x3e04041cu, 0x3e04042cu, 0x3e04043eu, 0x3e040c04u, 0x3e041c14u,
    0x3e042c14u, 0x3e0c1434u, 0x3e0c2404u, 0x3e140c14u, 0x3e14242cu, 0x3e142c14u, 0x3e1c0404u, 0x3e1c0c2cu,
    0x3e1c1c1cu, 0x3e1c3404u, 0x3e24140cu, 0x3e24240cu, 0x3e2c0404u, 0x3e2c0414u, 0x3e2c1424u, 0x3e341c04u,
};
static const int8_t orc_iq4nl_values[16] = {
    -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113,
};

static uint8_t orc_iq2_signs(uint32_t i7) {
    return (uint8_t)(i7 | ((uint32_t)(__builtin_popcount(i7) & 1) << 7));
}

/* IEEE half -> float (exact). */
static float orc_f16(const uint8_t* p) {
    const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
    const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t b;
    if (e == 31u) b = s | 0x7f800000u | (m << 13);
    else if (e != 0u) b = s | ((e + 112u) << 23) | (m << 13);
    else if (m == 0u) b = s;
    else {
        int ee = 113;
        uint32_t mm = m;
        while (!(mm & 1024u)) { mm <<= 1; --ee; }
        b = s | ((uint32_t)ee << 23) | ((mm & 1023u) << 13);
    }
    float f;
    memcpy(&f, &b, 4);
    return f;
}

int64_t orc_gguf_block_elems(uint32_t type) {
    switch (type) {
        case 0: case 1: return 1;
        case 8: return 32;
        case 11: case 12: case 13: case 14: case 18: case 23: return 256;
        default: return 0;
    }
}

int64_t orc_gguf_block_bytes(uint32_t type) {
    switch (type) {
        case 0: return 4;
        case 1: return 2;
        case 8: return 34;
        case 11: return 110;
        case 12: return 144;
        case 13: return 176;
        case 14: return 210;
        case 18: return 98;
        case 23: return 136;
        default: return 0;
    }
}

/* 6-bit scale and min j (0..7) of a Q4_K / Q5_K block (12 packed bytes):
 * src/gguf_quant.cpp:29-37. */
static void orc_k4_scale_min(const uint8_t* q, int j, int* sc, int* mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* Signed 6-bit scale i (0..15) of a Q3_K block: low 4 bits from bytes 0-7
 * (nibble i / 8 of byte i % 8), high 2 bits from bytes 8-11 (bits 2 (i / 4)
 * of byte 8 + i % 4); src/gguf_quant.cpp:109-121. */
static int orc_q3k_scale(const uint8_t* s12, int i) {
    const int lo = (s12[i % 8] >> (4 * (i / 8))) & 15;
    const int hi = (s12[8 + i % 4] >> (2 * (i / 4))) & 3;
    return (int)(int8_t)(uint8_t)(lo | (hi << 4));
}

float orc_gguf_value(uint32_t type, const uint8_t* b, int p) {
    switch (type) {
        case 0: { float f; memcpy(&f, b, 4); return f; }
        case 1: return orc_f16(b);
        case 8: /* d, 32 x int8 (src/gguf_quant.cpp:102-106) */
            return orc_f16(b) * (float)(int8_t)b[2 + p];
        case 11: { /* hmask[32] q[64] scales[12] d (src/gguf_quant.cpp:108-142) */
            const uint8_t* hmask = b;
            const uint8_t* q = b + 32;
            const int half = p / 128, r = p % 128, j = r / 32, sub = (r % 32) / 16, l = r % 16;
            const int idx = 16 * sub + l;
            const float d_all = orc_f16(b + 108);
            const float dl = d_all * (float)(orc_q3k_scale(b + 96, 8 * half + 2 * j + sub) - 32);
            const int v = (q[32 * half + idx] >> (2 * j)) & 3;
            const int hbit = hmask[idx] & (1 << (4 * half + j));
            return dl * (float)(v - (hbit ? 0 : 4));
        }
        case 12: case 13: { /* d dmin scales[12] (qh[32]) q[128] (src/gguf_quant.cpp:144-191) */
            const float d = orc_f16(b), dmin = orc_f16(b + 2);
            const int c64 = p / 64, c = p % 64, l = c % 32, hi = c / 32;
            int sc, mn;
            orc_k4_scale_min(b + 4, 2 * c64 + hi, &sc, &mn);
            const float d1 = d * (float)sc, m1 = dmin * (float)mn;
            const uint8_t* q = b + (type == 12 ? 16 : 48);
            int v = (q[32 * c64 + l] >> (4 * hi)) & 15;
            if (type == 13) v += (b[16 + l] & (1 << (2 * c64 + hi))) ? 16 : 0;
            return d1 * (float)v - m1;
        }
        case 14: { /* ql[128] qh[64] scales[16] d (src/gguf_quant.cpp:193-218) */
            const int n = p / 128, r = p % 128, quarter = r / 32, l = r % 32;
            const uint8_t* ql = b + 64 * n;
            const uint8_t* qh = b + 128 + 32 * n;
            const int8_t* sc = (const int8_t*)(b + 192) + 8 * n;
            const int lo = (ql[l + 32 * (quarter & 1)] >> (4 * (quarter >> 1))) & 15;
            const int q6 = (int)(int8_t)(uint8_t)(lo | (((qh[l] >> (2 * quarter)) & 3) << 4)) - 32;
            const float d = orc_f16(b + 208);
            return d * (float)sc[l / 16 + 2 * quarter] * (float)q6;
        }
        case 18: { /* d qs[64] signs+scales[32] (src/gguf_quant.cpp:220-239) */
            const int ib = p / 32, l = (p % 32) / 8, j = p % 8;
            const uint8_t* w = b + 66 + 4 * ib;
            const uint32_t aux = (uint32_t)w[0] | ((uint32_t)w[1] << 8) | ((uint32_t)w[2] << 16) |
                                 ((uint32_t)w[3] << 24);
            const float db = orc_f16(b) * (0.5f + (float)(aux >> 28)) * 0.5f;
            const uint8_t signs = orc_iq2_signs((aux >> (7 * l)) & 127u);
            const uint32_t g = orc_iq3xxs_grid[b[2 + 8 * ib + 2 * l + (j >> 2)]];
            const float mag = (float)((g >> (8 * (j & 3))) & 255u);
            return db * mag * ((signs & (1u << j)) ? -1.0f : 1.0f);
        }
        case 23: { /* d scales_h scales_l[4] qs[128] (src/gguf_quant.cpp:241-257) */
            const int ib = p / 32, c = p % 32;
            const uint16_t sh = (uint16_t)(b[2] | (b[3] << 8));
            const int lo = (b[4 + ib / 2] >> (4 * (ib & 1))) & 15;
            const int hi = (sh >> (2 * ib)) & 3;
            const int scale = (int)(int8_t)(uint8_t)(lo | (hi << 4)) - 32;
            const float dl = orc_f16(b) * (float)scale;
            const int code = (b[8 + 16 * ib + (c % 16)] >> (4 * (c / 16))) & 15;
            return dl * (float)orc_iq4nl_values[code];
        }
        default: return 0.0f;
    }
}

int orc_gguf_dequant_row(uint32_t type, const uint8_t* src, int64_t n, float* dst) {
    const int64_t be = orc_gguf_block_elems(type), bb = orc_gguf_block_bytes(type);
    if (!be || n % be) return -1;
    for (int64_t i = 0; i < n; ++i)
        dst[i] = orc_gguf_value(type, src + (i / be) * bb, (int)(i % be));
    return 0;
}

void orc_gguf_tables(const uint32_t** iq3xxs_grid, const int8_t** iq4nl_values) {
    *iq3xxs_grid = orc_iq3xxs_grid;
    *iq4nl_values = orc_iq4nl_values;
}

/* ---------------------------------------------------------------------------
 * GGUF int8-activation path (cuda/qgemm.cu:104-303, 556-587).
 * quantize_act_q8: per 32-element block, sx = absmax / 127 and
 * q = round-to-nearest-even(v * (1 / sx)) (q = 0 for an all-zero block).
 * A weight fragment of 8 elements is integers with one affine pair,
 * weight[j] = ds * wq[j] - dm (dm != 0 only for Q4_K / Q5_K); the dot of a
 * fragment with activations (xq, sx) is sx * (ds * sum(wq * xq) - dm * sum(xq)).
 * ------------------------------------------------------------------------- */
void orc_quant_act_q8(const float* x, int64_t n, int64_t in, int8_t* xq, float* xs) {
    for (int64_t t = 0; t < n; ++t)
        for (int64_t b = 0; b < in / 32; ++b) {
            const float* v = x + t * in + 32 * b;
            float amax = 0.0f;
            for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
            const float sx = amax / 127.0f;
            const float id = sx > 0.0f ? 1.0f / sx : 0.0f;
            for (int j = 0; j < 32; ++j) xq[t * in + 32 * b + j] = (int8_t)lrintf(v[j] * id);
            xs[t * (in / 32) + b] = sx;
        }
}

int orc_gguf_frag_i8(uint32_t type, const uint8_t* row, int64_t k, int8_t* wq, float* ds,
                     float* dm) {
    const int64_t be = orc_gguf_block_elems(type), bb = orc_gguf_block_bytes(type);
    if (!be || be == 1 || k % 8) return -1;
    const uint8_t* b = row + (k / be) * bb;
    const int p = (int)(k % be);
    *dm = 0.0f;
    switch (type) {
        case 8:
            *ds = orc_f16(b);
            for (int j = 0; j < 8; ++j) wq[j] = (int8_t)b[2 + p + j];
            return 0;
        case 11: {
            const int half = p / 128, r = p % 128, j = r / 32, sub = (r % 32) / 16, l = r % 16;
            *ds = orc_f16(b + 108) * (float)(orc_q3k_scale(b + 96, 8 * half + 2 * j + sub) - 32);
            for (int e = 0; e < 8; ++e) {
                const int idx = 16 * sub + l + e;
                const int v = (b[32 + 32 * half + idx] >> (2 * j)) & 3;
                wq[e] = (int8_t)(v - ((b[idx] & (1 << (4 * half + j))) ? 0 : 4));
            }
            return 0;
        }
        case 12: case 13: {
            const int c64 = p / 64, c = p % 64, l = c % 32, hi = c / 32;
            int sc, mn;
            orc_k4_scale_min(b + 4, 2 * c64 + hi, &sc, &mn);
            *ds = orc_f16(b) * (float)sc;
            *dm = orc_f16(b + 2) * (float)mn;
            const uint8_t* q = b + (type == 12 ? 16 : 48);
            for (int e = 0; e < 8; ++e) {
                int v = (q[32 * c64 + l + e] >> (4 * hi)) & 15;
                if (type == 13) v += (b[16 + l + e] & (1 << (2 * c64 + hi))) ? 16 : 0;
                wq[e] = (int8_t)v;
            }
            return 0;
        }
        case 14: {
            const int nn = p / 128, r = p % 128, quarter = r / 32, l = r % 32;
            const uint8_t* ql = b + 64 * nn;
            const uint8_t* qh = b + 128 + 32 * nn;
            *ds = orc_f16(b + 208) * (float)((const int8_t*)(b + 192))[8 * nn + l / 16 + 2 * quarter];
            for (int e = 0; e < 8; ++e) {
                const int lo = (ql[l + e + 32 * (quarter & 1)] >> (4 * (quarter >> 1))) & 15;
                wq[e] = (int8_t)((int)(lo | (((qh[l + e] >> (2 * quarter)) & 3) << 4)) - 32);
            }
            return 0;
        }
        case 18: {
            const int ib = p / 32, l = (p % 32) / 8;
            const uint8_t* w = b + 66 + 4 * ib;
            const uint32_t aux = (uint32_t)w[0] | ((uint32_t)w[1] << 8) | ((uint32_t)w[2] << 16) |
                                 ((uint32_t)w[3] << 24);
            *ds = orc_f16(b) * (0.5f + (float)(aux >> 28)) * 0.5f;
            const uint8_t signs = orc_iq2_signs((aux >> (7 * l)) & 127u);
            for (int e = 0; e < 8; ++e) {
                const uint32_t g = orc_iq3xxs_grid[b[2 + 8 * ib + 2 * l + (e >> 2)]];
                const int mag = (int)((g >> (8 * (e & 3))) & 255u);
                wq[e] = (int8_t)((signs & (1u << e)) ? -mag : mag);
            }
            return 0;
        }
        case 23: {
            const int ib = p / 32, c = p % 32;
            const uint16_t sh = (uint16_t)(b[2] | (b[3] << 8));
            const int lo = (b[4 + ib / 2] >> (4 * (ib & 1))) & 15;
            const int hi = (sh >> (2 * ib)) & 3;
            *ds = orc_f16(b) * (float)((int)(int8_t)(uint8_t)(lo | (hi << 4)) - 32);
            for (int e = 0; e < 8; ++e) {
                const int cc = c + e;
                wq[e] = orc_iq4nl_values[(b[8 + 16 * ib + (cc % 16)] >> (4 * (cc / 16))) & 15];
            }
            return 0;
        }
        default: return -1;
    }
}

int orc_gemm_q_i8(uint32_t type, const int8_t* xq, const float* xs, const uint8_t* w, int64_t n,
                  int64_t in, int64_t out, int64_t row_bytes, double* y) {
    for (int64_t o = 0; o < out; ++o)
        for (int64_t t = 0; t < n; ++t) {
            double acc = 0.0;
            for (int64_t k = 0; k < in; k += 8) {
                int8_t wq[8];
                float ds, dm;
                if (orc_gguf_frag_i8(type, w + o * row_bytes, k, wq, &ds, &dm)) return -1;
                int sumi = 0, sumx = 0;
                for (int j = 0; j < 8; ++j) {
                    sumi += (int)wq[j] * (int)xq[t * in + k + j];
                    sumx += (int)xq[t * in + k + j];
                }
                acc += (double)xs[t * (in / 32) + k / 32] *
                       ((double)ds * (double)sumi - (double)dm * (double)sumx);
            }
            y[t * out + o] = acc;
        }
    return 0;
}
