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
// Each candidate is one 64-bit key whose unsigned order is the selection
// order of cuda/moe_router.cu:48-53: high word = choose mapped to a
// monotone unsigned code (NaN just above "no candidate", below every number),
// low word = ~expert, so equal choose values prefer the lower expert index.
// Each of the k rounds: every lane offers its best untaken key; a max over
// each 16-lane row with DPP row rotations (VALU latency, no LDS round trip),
// then the 4 row maxima via readlane and a scalar max. The owner lane of
// the winner retires it. Every lane sees the same winner (a uniform value).
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

__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ e_bias, int n, int E, int topk,
    int norm_topk, float routed_scale, int* __restrict__ topk_ids, float* __restrict__ topk_w) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;   // whole wave
    const float* lt = logits + (size_t)t * E;
    float score[kMaxPerLane];
    uint32_t ch[kMaxPerLane];   // order codes, 0 = no candidate / taken
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
        const int e = lane + 64 * j;
        score[j] = 0.0f;
        ch[j] = 0u;
        if (e < E) {
            const float sc = sigmoid_fixed(lt[e]);
            score[j] = sc;
            ch[j] = order_code(sc + (e_bias ? e_bias[e] : 0.0f));
        }
    }
    float wsel[8];
    int idsel[8];
    float wsum = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        if (k >= topk) break;
        // Lane-local best (ascending j == ascending expert; strict > keeps lower).
        uint32_t h = 0u, l = 0u;
#pragma unroll
        for (int j = 0; j < kMaxPerLane; ++j)
            kmax(h, l, ch[j], ch[j] ? ~(uint32_t)(lane + 64 * j) : 0u);
        // Row max (row_ror:1,2,4,8 over 16 lanes), then across the 4 rows.
        kmax_dpp<0x121>(h, l);
        kmax_dpp<0x122>(h, l);
        kmax_dpp<0x124>(h, l);
        kmax_dpp<0x128>(h, l);
        uint32_t bh = (uint32_t)__builtin_amdgcn_readlane((int)h, 0);
        uint32_t bl = (uint32_t)__builtin_amdgcn_readlane((int)l, 0);
        kmax(bh, bl, (uint32_t)__builtin_amdgcn_readlane((int)h, 16),
             (uint32_t)__builtin_amdgcn_readlane((int)l, 16));
        kmax(bh, bl, (uint32_t)__builtin_amdgcn_readlane((int)h, 32),
             (uint32_t)__builtin_amdgcn_readlane((int)l, 32));
        kmax(bh, bl, (uint32_t)__builtin_amdgcn_readlane((int)h, 48),
             (uint32_t)__builtin_amdgcn_readlane((int)l, 48));
        const int e = (int)~bl;               // uniform winner
        const int owner = e & 63, jw = e >> 6;
        float sw = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxPerLane; ++j) {
            if (j == jw) {
                sw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(score[j]), owner));
                if (lane == owner) ch[j] = 0u;
            }
        }
        idsel[k] = e;
        wsel[k] = sw;
        wsum = wsum + sw;
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
