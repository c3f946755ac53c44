// Wave64 top-k selection shared by the router kernels and the gate/up
// kernel's small-batch routing prologue.
//
// Reference: cuda/moe_router.cu:17-79 (sigmoid scores, + correction bias,
// k rounds of the largest choose value, normalised weights times the
// routed scale).
#pragma once
#include "common.hpp"

namespace glmmoe {

// ---------------------------------------------------------------------------
// Top-k. One wave per token; lane l owns experts l, l+64, ... (E <= 512).
// Each candidate is one 64-bit key whose unsigned order is the selection
// order of cuda/moe_router.cu:48-53: high word = choose mapped to a
// monotone unsigned code (NaN just above "no candidate", below every number),
// low word = ~expert, so equal choose values prefer the lower expert index.
// kmax / kmax_dpp: a max over keys (each 16-lane row with DPP row rotations,
// then the 4 row maxima via readlane), used where one key per wave is wanted.
// ---------------------------------------------------------------------------
constexpr int kMaxPerLane = 8;  // E <= 512

__device__ __forceinline__ uint32_t order_code(float f) {
    if (f != f) return 1u;
    if (f == 0.0f) f = 0.0f;   // -0 == +0: equal values fall through to the index
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ void kmax(uint32_t& h, uint32_t& l, uint32_t oh, uint32_t ol) {
    const bool take = oh > h || (oh == h && ol > l);
    h = take ? oh : h;
    l = take ? ol : l;
}

template <int CTRL>
__device__ __forceinline__ void kmax_dpp(uint32_t& h, uint32_t& l) {
    const uint32_t oh = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)h, CTRL, 0xf, 0xf, false);
    const uint32_t ol = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)l, CTRL, 0xf, 0xf, false);
    kmax(h, l, oh, ol);
}

// Unsigned maximum over the wave, uniform: within each 16-lane row by DPP
// row rotations, then the 4 row maxima.
template <int CTRL>
__device__ __forceinline__ uint32_t umax_dpp(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
    return o > v ? o : v;
}
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
    v = umax_dpp<0x121>(v);
    v = umax_dpp<0x122>(v);
    v = umax_dpp<0x124>(v);
    v = umax_dpp<0x128>(v);
    uint32_t m = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
#pragma unroll
    for (int r = 1; r < 4; ++r) {
        const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)v, 16 * r);
        m = o > m ? o : m;
    }
    return m;
}

constexpr int kTopkScratch = 40;   // LDS words per wave for topk_wave

// Selection for token row lt (one wave; every lane calls it): the k rounds of
// cuda/moe_router.cu:48-53 over keys (order code of choose, ~expert), each
// lane's keys pre-sorted so a round looks at one head per lane. scratch is
// unused (kept for the callers' LDS layout). COH: read the logits (or codes
// and scores) with device-coherent loads and store ids/weights with
// device-coherent stores. ids_out / w_out may be null (then only ids_copy,
// when given, receives the ids).
template <bool COH, int NJ>
__device__ __forceinline__ void topk_wave_nj(const float* __restrict__ lt,
                                          const float* __restrict__ e_bias, int E, int topk,
                                          int norm_topk, float routed_scale,
                                          int* __restrict__ ids_out, float* __restrict__ w_out,
                                          uint32_t* scratch, const uint32_t* pcode,
                                          const float* pscore, int* ids_copy = nullptr) {
    const int lane = threadIdx.x & 63;
    float score[NJ];
    uint32_t ch[NJ];   // order codes, 0 = no candidate
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int e = lane + 64 * j;
        score[j] = 0.0f;
        ch[j] = 0u;
        if (e < E) {
            if (pcode) {   // codes and scores already computed by the caller
                ch[j] = COH ? ld_dev(pcode + e) : pcode[e];
                score[j] = COH ? ld_dev(pscore + e) : pscore[e];
            } else {
                const float sc = sigmoid_fixed(COH ? ld_dev(lt + e) : lt[e]);
                score[j] = sc;
                ch[j] = order_code(sc + (e_bias ? e_bias[e] : 0.0f));
            }
        }
    }
    // 1. Keys (order code, ~expert): a larger key is chosen first; equal
    //    codes prefer the lower expert. Each lane sorts its NJ keys, largest
    //    first, scores alongside (a fixed compare-exchange network).
    uint32_t kl[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) kl[j] = ch[j] ? ~(uint32_t)(lane + 64 * j) : 0u;
#pragma unroll
    for (int i = 0; i < NJ; ++i)
#pragma unroll
        for (int j = 0; j + 1 < NJ - i; ++j) {
            const bool up = ch[j + 1] > ch[j] || (ch[j + 1] == ch[j] && kl[j + 1] > kl[j]);
            const uint32_t h0 = ch[j], l0 = kl[j];
            const float s0 = score[j];
            ch[j] = up ? ch[j + 1] : ch[j];
            kl[j] = up ? kl[j + 1] : kl[j];
            score[j] = up ? score[j + 1] : score[j];
            ch[j + 1] = up ? h0 : ch[j + 1];
            kl[j + 1] = up ? l0 : kl[j + 1];
            score[j + 1] = up ? s0 : score[j + 1];
        }
    // 2. k rounds, as cuda/moe_router.cu:48-53 does them: the largest lane
    //    head over the wave (a max over each 16-lane row with DPP row
    //    rotations, then the 4 row maxima); the owner lane drops its head.
    //    Lane k keeps round k's pick. (A rolled loop: these kernels run
    //    once per call, where fetching unrolled code costs more than the
    //    loop.)
    float wsel = 0.0f;
    int idsel = 0;
    float wsum = 0.0f;
#pragma unroll 1
    for (int k = 0; k < topk; ++k) {
        // The largest head key (code, ~expert): the largest code over the
        // wave, then the largest ~expert among the heads holding that code.
        const uint32_t bh = wave_umax(ch[0]);
        const uint32_t bl = wave_umax(ch[0] == bh ? kl[0] : 0u);
        const int e = (int)~bl;               // uniform winner
        const int owner = e & 63;
        const float sw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(score[0]), owner));
        if (lane == owner) {
#pragma unroll
            for (int j = 0; j + 1 < NJ; ++j) {
                ch[j] = ch[j + 1];
                kl[j] = kl[j + 1];
                score[j] = score[j + 1];
            }
            ch[NJ - 1] = 0u;
            kl[NJ - 1] = 0u;
        }
        idsel = lane == k ? e : idsel;
        wsel = lane == k ? sw : wsel;
        wsum = wsum + sw;
    }
    // 3. Weights in selection order, normalized by their sum in that order.
    (void)scratch;
    if (lane < topk) {
        float v = wsel;
        if (norm_topk && wsum > 0.0f) v = v / wsum;
        // ids_out == nullptr: only the copy (a caller that needs the ids alone).
        if (ids_out && COH) {
            st_dev(ids_out + lane, idsel);
            st_dev(w_out + lane, v * routed_scale);
        } else if (ids_out) {
            ids_out[lane] = idsel;
            w_out[lane] = v * routed_scale;
        }
        if (ids_copy) ids_copy[lane] = idsel;
    }
}

}  // namespace glmmoe
