// Router: bf16 router-logit GEMM in a fixed reduction order, and the
// wave64 sigmoid + bias top-k selection.
//
// Reference: src/model_gpu.cpp:1448-1450 (gemm_linear on the router, then
// moe_router), cuda/moe_router.cu:17-79, src/model_glm52.cpp:1105-1129.
#include "common.hpp"
#include "kernels.hpp"

namespace glmmoe {

// ---------------------------------------------------------------------------
// Router logits. One wave per (expert, group of 8 tokens). Lane c owns K
// chunk c (128 consecutive inputs) and keeps 8 independent running sums, one
// per token, each accumulated from zero in ascending K. The chunk sums of a
// token are then added in ascending chunk order by one lane. That is exactly
// the order the CPU oracle restates (chunked linear_forward), and since bf16
// products are exact in fp32, fma(x, w, s) == s + x*w, so logits are
// bit-identical to it.
// ---------------------------------------------------------------------------
constexpr int kRouterTG = 8;    // tokens per wave
constexpr int kRouterKC = 128;  // K chunk
constexpr int kRouterMaxChunks = 64;

__global__ __launch_bounds__(256) void router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr, int n, int H, int E,
    float* __restrict__ logits, float* __restrict__ xsum) {
    __shared__ float part[4][kRouterTG][kRouterMaxChunks + 1];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const long wid = (long)blockIdx.x * 4 + wv;
    const int ngroups = (n + kRouterTG - 1) / kRouterTG;
    // Waves past the end stay resident until the barrier (no early return).
    const bool active = wid < (long)E * ngroups;
    const int e = active ? (int)(wid % E) : 0;
    const int t0 = active ? (int)(wid / E) * kRouterTG : n;
    const int nchunks = (H + kRouterKC - 1) / kRouterKC;

    if (active && lane < nchunks) {
        const int k0 = lane * kRouterKC;
        const int klen = min(kRouterKC, H - k0);  // multiple of 8
        float s[kRouterTG];
        float xs[kRouterTG];
#pragma unroll
        for (int t = 0; t < kRouterTG; ++t) { s[t] = 0.0f; xs[t] = 0.0f; }
        const uint4* wp = reinterpret_cast<const uint4*>(wr + (size_t)e * H + k0);
        for (int i8 = 0; i8 < klen / 8; ++i8) {
            const uint4 wv4 = wp[i8];
            const uint32_t wd[4] = {wv4.x, wv4.y, wv4.z, wv4.w};
#pragma unroll
            for (int t = 0; t < kRouterTG; ++t) {
                if (t0 + t >= n) break;
                const uint4 xv4 =
                    reinterpret_cast<const uint4*>(x + (size_t)(t0 + t) * H + k0)[i8];
                const uint32_t xd[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float xl = bf16_to_f32(xd[j] & 0xffffu), xh = bf16_to_f32(xd[j] >> 16);
                    const float wl = bf16_to_f32(wd[j] & 0xffffu), wh = bf16_to_f32(wd[j] >> 16);
                    s[t] = __builtin_fmaf(xl, wl, s[t]);
                    s[t] = __builtin_fmaf(xh, wh, s[t]);
                    if (e == 0 && xsum) { xs[t] += xl; xs[t] += xh; }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kRouterTG; ++t) {
            part[wv][t][lane] = s[t];
            if (e == 0 && xsum && t0 + t < n) xsum[(size_t)(t0 + t) * nchunks + lane] = xs[t];
        }
    }
    __syncthreads();
    if (active && lane < kRouterTG && t0 + lane < n) {
        float total = 0.0f;
        for (int c = 0; c < nchunks; ++c) total = total + part[wv][lane][c];
        logits[(size_t)(t0 + lane) * E + e] = total;
    }
}

// Activation group sums alone (for callers that bring their own routing).
__global__ __launch_bounds__(256) void xsum_kernel(const uint16_t* __restrict__ x, int n,
                                                   int H, float* __restrict__ xsum) {
    const int nchunks = H / kRouterKC;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n * nchunks) return;
    const int t = (int)(i / nchunks), c = (int)(i % nchunks);
    const uint4* p = reinterpret_cast<const uint4*>(x + (size_t)t * H + c * kRouterKC);
    float s = 0.0f;
    for (int j = 0; j < kRouterKC / 8; ++j) {
        const uint4 v = p[j];
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) { s += bf16_to_f32(d[q] & 0xffffu); s += bf16_to_f32(d[q] >> 16); }
    }
    xsum[i] = s;
}

// ---------------------------------------------------------------------------
// Top-k. One wave per token; lane l owns experts l, l+64, ... (E <= 512).
// Candidate order: finite/inf choose values descending, ties to the lower
// expert index (cuda/moe_router.cu:48-53), NaN after every number. Each of
// the k rounds takes a lane-local best (ascending expert order, strict >),
// then a butterfly arg-max across the wave; the total order makes every lane
// agree on the winner.
// ---------------------------------------------------------------------------
constexpr int kMaxPerLane = 8;  // E <= 512

struct Cand {
    float c;   // choose
    float s;   // unbiased score
    int e;     // expert id, INT_MAX when none
    int cls;   // 2 = number, 1 = NaN, 0 = none
};

__device__ __forceinline__ bool better(const Cand& a, const Cand& b) {
    if (a.cls != b.cls) return a.cls > b.cls;
    if (a.cls == 2 && a.c != b.c) return a.c > b.c;
    return a.e < b.e;
}

__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ e_bias, int n, int E, int topk,
    int norm_topk, float routed_scale, int* __restrict__ topk_ids, float* __restrict__ topk_w) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;
    const float* lt = logits + (size_t)t * E;
    float score[kMaxPerLane], choose[kMaxPerLane];
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
        const int e = lane + 64 * j;
        if (e < E) {
            const float sc = sigmoid_fixed(lt[e]);
            score[j] = sc;
            choose[j] = sc + (e_bias ? e_bias[e] : 0.0f);
            cnt = j + 1;
        } else {
            score[j] = 0.0f;
            choose[j] = 0.0f;
        }
    }
    uint32_t taken = 0;
    float wsel[8];
    int idsel[8];
    float wsum = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        if (k >= topk) break;
        Cand best{0.0f, 0.0f, 0x7fffffff, 0};
#pragma unroll
        for (int j = 0; j < kMaxPerLane; ++j) {
            if (j < cnt && !((taken >> j) & 1u)) {
                Cand c{choose[j], score[j], lane + 64 * j, (choose[j] != choose[j]) ? 1 : 2};
                if (better(c, best)) best = c;
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            Cand o;
            o.c = __shfl_xor(best.c, off);
            o.s = __shfl_xor(best.s, off);
            o.e = __shfl_xor(best.e, off);
            o.cls = __shfl_xor(best.cls, off);
            if (better(o, best)) best = o;
        }
        if ((best.e & 63) == lane) taken |= 1u << (best.e >> 6);
        idsel[k] = best.e;
        wsel[k] = best.s;
        wsum = wsum + best.s;
    }
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (k >= topk) break;
            float v = wsel[k];
            if (norm_topk && wsum > 0.0f) v = v / wsum;
            topk_ids[(size_t)t * topk + k] = idsel[k];
            topk_w[(size_t)t * topk + k] = v * routed_scale;
        }
    }
}

int launch_router_logits(const uint16_t* x, const uint16_t* wr, int n, int H, int E,
                         float* logits, float* xsum, hipStream_t s) {
    const long waves = (long)E * ((n + kRouterTG - 1) / kRouterTG);
    const long blocks = (waves + 3) / 4;
    hipLaunchKernelGGL(router_logits_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, wr, n,
                       H, E, logits, xsum);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_xsum(const uint16_t* x, int n, int H, float* xsum, hipStream_t s) {
    const long items = (long)n * (H / kRouterKC);
    hipLaunchKernelGGL(xsum_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, x,
                       n, H, xsum);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_router_topk(const float* logits, const float* e_bias, int n, int E, int topk,
                       int norm_topk, float routed_scale, int* ids, float* w, hipStream_t s) {
    hipLaunchKernelGGL(router_topk_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s,
                       logits, e_bias, n, E, topk, norm_topk, routed_scale, ids, w);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace glmmoe
