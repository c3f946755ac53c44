// Reference-signature kernels: the launchers of glmserve's cuda/kernels.cuh
// that the MoE branch of the forward calls besides the grouped experts, with
// the reference's arguments, layouts and fp32 activations.
//
//   ref_gemm_w4_kernel    gemm_w4a16  (cuda/kernels.cuh:50-52, cuda/int4_gemm.cu:15-48):
//                         y[n,out] = x[n,in] . W^T (+ bias), W int4 from qW [out, ceil(in/2)]
//                         (low nibble = even column, value nibble - 8) and fp32 scales
//                         [out, ceil(in/g)]. The shared expert's three linears.
//   ref_gemm_fp8_kernel   gemm_fp8    (cuda/kernels.cuh:55-57, cuda/fp8_gemm.cu:14-44):
//                         W e4m3 [out, in] with an optional fp32 scale per row.
//   ref_expert_f32_kernel moe_expert_ffn (cuda/kernels.cuh:252-257, cuda/moe_expert.cu:32-130):
//                         routed experts with fp32 weights; out overwritten with
//                         sum_s w[t,s] * down_e(silu(gate_e x) * up_e x), slot order.
//   silu_mul / add_inplace (cuda/kernels.cuh:281-282, cuda/mla_glue.cu:10-28).
//   f32_to_bf16           activations for the bf16 grouped kernels behind the
//                         reference-signature moe_expert_ffn_w4a16.
//
// The GEMVs are decode-shaped (the shared expert at small n): a workgroup of 4
// waves owns 16 output rows (4 per wave) and walks the tokens in blocks of 8.
// Each 512-wide K chunk of the 8 token rows is staged once in LDS and shared
// by the 4 waves; each lane then holds 8 consecutive K of its 4 rows (one
// dword of int4 codes, or 8 e4m3 bytes, per row) and accumulates 4 x 8 dot
// products in fp32. Lane partials are combined by a fixed xor butterfly, so
// results are deterministic. Weights are read once per token block.
#include "common.hpp"
#include "kernels.hpp"

namespace glmmoe {

constexpr int kGvRows = 16;   // output rows per workgroup (4 per wave)
constexpr int kGvTok = 8;     // tokens per block
constexpr int kGvKC = 512;    // K per staged chunk (64 lanes x 8)

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

// OCP e4m3 ("fn"): bias 7, no infinities, 0x7f / 0xff are NaN.
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
    const uint32_t s = (c & 0x80u) << 24, e = (c >> 3) & 15u, m = c & 7u;
    if (e == 15u && m == 7u) return __uint_as_float(s | 0x7fc00000u);
    if (e == 0u) return __uint_as_float(s) + (s ? -1.0f : 1.0f) * (float)m * 0.001953125f;  // m * 2^-9
    return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

// Weight decode of 8 consecutive K of one row: W4 (one dword of codes and the
// group's scale) or FP8 (two dwords of e4m3 and the row scale).
template <bool FP8>
struct GvRow {
    uint32_t w0, w1;
    float s;
    __device__ __forceinline__ float at(int j) const {
        if constexpr (FP8) {
            const uint32_t d = j < 4 ? w0 : w1;
            return e4m3_to_f32((d >> (8 * (j & 3))) & 0xffu) * s;
        } else {
            return (float)((int)((w0 >> (4 * j)) & 15u) - 8) * s;
        }
    }
};

// Vector path: in % 8 == 0 and (W4) group % 8 == 0, so a lane's 8 K share one
// scale and one aligned dword (W4) or two (FP8) per row.
template <bool FP8>
__global__ __launch_bounds__(256) void ref_gemv_kernel(const float* __restrict__ x,
                                                       const uint8_t* __restrict__ w,
                                                       const float* __restrict__ sc,
                                                       const float* __restrict__ bias,
                                                       float* __restrict__ y, int n, int in,
                                                       int out, int g) {
    __shared__ __align__(16) float xs[kGvTok][kGvKC];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int o0 = blockIdx.x * kGvRows + wave * 4;
    const size_t rstride = FP8 ? (size_t)in : (size_t)(in + 1) / 2;   // bytes per weight row
    const int ng = FP8 ? 1 : (in + g - 1) / g;
    for (int t0 = 0; t0 < n; t0 += kGvTok) {
        const int nt = min(kGvTok, n - t0);
        float acc[4][kGvTok];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < kGvTok; ++t) acc[r][t] = 0.0f;
        for (int k0 = 0; k0 < in; k0 += kGvKC) {
            const int kc = min(kGvKC, in - k0);
            __syncthreads();
            for (int i = threadIdx.x; i < kGvTok * (kGvKC / 4); i += blockDim.x) {
                const int t = i / (kGvKC / 4), c4 = i % (kGvKC / 4);
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (t < nt && 4 * c4 < kc)
                    v = *reinterpret_cast<const float4*>(x + (size_t)(t0 + t) * in + k0 + 4 * c4);
                *reinterpret_cast<float4*>(&xs[t][4 * c4]) = v;
            }
            __syncthreads();
            const int kk = lane * 8;
            if (kk < kc) {
                GvRow<FP8> row[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int o = min(o0 + r, out - 1);
                    const uint8_t* wr = w + (size_t)o * rstride;
                    const int k = k0 + kk;
                    if constexpr (FP8) {
                        const uint2 d = *reinterpret_cast<const uint2*>(wr + k);
                        row[r].w0 = d.x;
                        row[r].w1 = d.y;
                        row[r].s = sc ? sc[o] : 1.0f;
                    } else {
                        row[r].w0 = *reinterpret_cast<const uint32_t*>(wr + k / 2);
                        row[r].w1 = 0u;
                        row[r].s = sc[(size_t)o * ng + k / g];
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float wv[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) wv[r] = row[r].at(j);
#pragma unroll
                    for (int t = 0; t < kGvTok; ++t) {
                        const float xv = xs[t][kk + j];
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[r][t] = __builtin_fmaf(wv[r], xv, acc[r][t]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < kGvTok; ++t) {
                const float v = wave_sum(acc[r][t]);
                const int o = o0 + r;
                if (lane == 0 && t < nt && o < out)
                    y[(size_t)(t0 + t) * out + o] = bias ? v + bias[o] : v;
            }
    }
}

// Any shape: one K position per lane step, no staging (the layouts of
// cuda/int4_gemm.cu:20-30 with an odd in or a group size not a multiple of 8).
template <bool FP8>
__global__ __launch_bounds__(256) void ref_gemv_any_kernel(const float* __restrict__ x,
                                                           const uint8_t* __restrict__ w,
                                                           const float* __restrict__ sc,
                                                           const float* __restrict__ bias,
                                                           float* __restrict__ y, int n, int in,
                                                           int out, int g) {
    const int lane = threadIdx.x & 63;
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= out) return;
    const size_t rstride = FP8 ? (size_t)in : (size_t)(in + 1) / 2;
    const int ng = FP8 ? 1 : (in + g - 1) / g;
    const uint8_t* wr = w + (size_t)o * rstride;
    for (int t = 0; t < n; ++t) {
        const float* xt = x + (size_t)t * in;
        float acc = 0.0f;
        for (int k = lane; k < in; k += 64) {
            float wv;
            if constexpr (FP8) {
                wv = e4m3_to_f32(wr[k]) * (sc ? sc[o] : 1.0f);
            } else {
                const uint32_t b = wr[k >> 1];
                wv = (float)((int)((k & 1) ? (b >> 4) : (b & 15u)) - 8) * sc[(size_t)o * ng + k / g];
            }
            acc = __builtin_fmaf(wv, xt[k], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) y[(size_t)t * out + o] = bias ? acc + bias[o] : acc;
    }
}

template <bool FP8>
static int launch_ref_gemv(const float* x, const uint8_t* w, const float* sc, const float* bias,
                           float* y, int n, int in, int out, int g, hipStream_t s) {
    const bool vec = in % 8 == 0 && (FP8 || g % 8 == 0);
    if (vec)
        hipLaunchKernelGGL(ref_gemv_kernel<FP8>, dim3((unsigned)((out + kGvRows - 1) / kGvRows)),
                           dim3(256), 0, s, x, w, sc, bias, y, n, in, out, g);
    else
        hipLaunchKernelGGL(ref_gemv_any_kernel<FP8>, dim3((unsigned)((out + 3) / 4)), dim3(256), 0,
                           s, x, w, sc, bias, y, n, in, out, g);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_ref_gemm_w4(const float* x, const uint8_t* qw, const float* sc, const float* bias,
                       float* y, int n, int in, int out, int g, hipStream_t s) {
    return launch_ref_gemv<false>(x, qw, sc, bias, y, n, in, out, g, s);
}

int launch_ref_gemm_fp8(const float* x, const uint8_t* w, const float* sc, const float* bias,
                        float* y, int n, int in, int out, hipStream_t s) {
    return launch_ref_gemv<true>(x, w, sc, bias, y, n, in, out, 1, s);
}

// ---------------------------------------------------------------------------
// fp32-weight routed experts, one workgroup (8 waves) per token: the k rows
// h_s = silu(Wg_e x) * (Wu_e x) of the token's experts go to LDS, then each
// output feature o is sum_s w_s * (Wd_e[o] . h_s) in slot order. Every dot
// product is one wave: lanes over K, then the xor butterfly.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + expf(-v)); }

__device__ __forceinline__ float wave_dot(const float* a, const float* b, int len, int lane) {
    float acc = 0.0f;
    if ((len & 3) == 0) {
        for (int i = 4 * lane; i < len; i += 256) {
            const float4 u = *reinterpret_cast<const float4*>(a + i);
            const float4 v = *reinterpret_cast<const float4*>(b + i);
            acc = __builtin_fmaf(u.x, v.x, acc);
            acc = __builtin_fmaf(u.y, v.y, acc);
            acc = __builtin_fmaf(u.z, v.z, acc);
            acc = __builtin_fmaf(u.w, v.w, acc);
        }
    } else {
        for (int i = lane; i < len; i += 64) acc = __builtin_fmaf(a[i], b[i], acc);
    }
    return wave_sum(acc);
}

__global__ __launch_bounds__(512) void ref_expert_f32_kernel(
    const float* __restrict__ x, const int* __restrict__ ids, const float* __restrict__ wts,
    const float* __restrict__ gw, const float* __restrict__ uw, const float* __restrict__ dw,
    int topk, int H, int I, float* __restrict__ out) {
    extern __shared__ __align__(16) float hbuf[];   // [topk][I]
    const int t = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const float* xt = x + (size_t)t * H;
    for (int r = wave; r < topk * I; r += nw) {
        const int s = r / I, f = r % I;
        const size_t e = (size_t)ids[(size_t)t * topk + s];
        const float gv = wave_dot(gw + (e * I + f) * H, xt, H, lane);
        const float uv = wave_dot(uw + (e * I + f) * H, xt, H, lane);
        if (lane == 0) hbuf[r] = silu_f32(gv) * uv;
    }
    __syncthreads();
    for (int o = wave; o < H; o += nw) {
        float acc = 0.0f;
        for (int s = 0; s < topk; ++s) {
            const size_t e = (size_t)ids[(size_t)t * topk + s];
            const float d = wave_dot(dw + (e * H + o) * I, hbuf + (size_t)s * I, I, lane);
            acc = acc + wts[(size_t)t * topk + s] * d;
        }
        if (lane == 0) out[(size_t)t * H + o] = acc;
    }
}

int launch_ref_expert_f32(const float* x, const int* ids, const float* w, const float* gw,
                          const float* uw, const float* dw, int n, int topk, int H, int I,
                          float* out, hipStream_t s) {
    const size_t lds = (size_t)topk * I * 4;
    if (lds > 160 * 1024) return -2;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&ref_expert_f32_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) !=
            hipSuccess)
            return -4;
        attr_set = true;
    }
    hipLaunchKernelGGL(ref_expert_f32_kernel, dim3((unsigned)n), dim3(512), lds, s, x, ids, w, gw,
                       uw, dw, topk, H, I, out);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// ---------------------------------------------------------------------------
// Elementwise glue.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ref_silu_mul_kernel(const float* __restrict__ g,
                                                           const float* __restrict__ u,
                                                           float* __restrict__ o, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = silu_f32(g[i]) * u[i];
}

__global__ __launch_bounds__(256) void ref_add_inplace_kernel(float* __restrict__ y,
                                                              const float* __restrict__ x, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] += x[i];
}

__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float* __restrict__ x,
                                                          uint16_t* __restrict__ y, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (uint16_t)f32_to_bf16(x[i]);
}

static unsigned blocks_for(long n) { return (unsigned)((n + 255) / 256); }

int launch_ref_silu_mul(const float* g, const float* u, float* o, long n, hipStream_t s) {
    hipLaunchKernelGGL(ref_silu_mul_kernel, dim3(blocks_for(n)), dim3(256), 0, s, g, u, o, n);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_ref_add_inplace(float* y, const float* x, long n, hipStream_t s) {
    hipLaunchKernelGGL(ref_add_inplace_kernel, dim3(blocks_for(n)), dim3(256), 0, s, y, x, n);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_f32_to_bf16(const float* x, uint16_t* y, long n, hipStream_t s) {
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(blocks_for(n)), dim3(256), 0, s, x, y, n);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace glmmoe
