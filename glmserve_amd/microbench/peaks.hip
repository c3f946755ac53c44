// Measured peaks of the MI355X this library runs on, the denominators of the
// roofline fractions: dense MFMA rate (bf16 and fp16 32x32x16, fp8 32x32x64
// with block scales), the s_memtime rate the MFMA waves see, and HBM read and
// copy bandwidth. Prints one JSON line. Built by glmserve_amd/build.py into
// glmserve_amd/_lib/glmmoe_peaks; run it on the GPU box:
//   ./glmserve_amd/_lib/glmmoe_peaks
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

__device__ unsigned long long g_ticks[1];

// 8 waves per CU, 4 independent accumulator chains per wave (enough to keep
// the MFMA pipe of each SIMD busy). KIND 0 bf16, 1 fp16, 2 fp8 (scaled).
template <int KIND>
__global__ __launch_bounds__(512) void mfma_kernel(float* out, int iters) {
    f32x16 c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) c[j][e] = 0.0f;
    bf16x8 ab;
    f16x8 ah;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        ab[i] = (__bf16)(threadIdx.x * 1e-3f + i);
        ah[i] = (_Float16)(threadIdx.x * 1e-3f + i);
    }
    i32x8 a8;
#pragma unroll
    for (int i = 0; i < 8; ++i) a8[i] = (int)(0x38383838u + threadIdx.x + i);
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (KIND == 0) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ab, ab, c[j], 0, 0, 0);
            else if constexpr (KIND == 1) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ah, c[j], 0, 0, 0);
            else c[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, a8, c[j], 0, 0, 0, 127, 0, 127);
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) s += c[j][0] + c[j][15];
    out[blockIdx.x * 512 + threadIdx.x] = s;
    if (blockIdx.x == 0 && threadIdx.x == 0) g_ticks[0] = t1 - t0;
}

// Streaming read: every byte of src once per launch, 16 B per lane per load.
__global__ __launch_bounds__(256) void read_kernel(const uint4* __restrict__ src, size_t n16,
                                                   uint4* __restrict__ sink) {
    uint4 acc = {0, 0, 0, 0};
    for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) {
        const uint4 v = src[i];
        acc.x ^= v.x;
        acc.y ^= v.y;
        acc.z ^= v.z;
        acc.w ^= v.w;
    }
    if ((acc.x & acc.y & acc.z & acc.w) == 0xdeadbeefu) sink[threadIdx.x] = acc;
}
__global__ __launch_bounds__(256) void copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                   size_t n16) {
    for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

#define CK(x)                                                  \
    do {                                                       \
        if ((x) != hipSuccess) {                               \
            fprintf(stderr, "HIP error at %s\n", #x);          \
            return 1;                                          \
        }                                                      \
    } while (0)

template <class F>
static float time_ms(F launch, int reps) {
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    launch();
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(e0);
    for (int r = 0; r < reps; ++r) launch();
    (void)hipEventRecord(e1);
    (void)hipEventSynchronize(e1);
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return ms / reps;
}

int main() {
    int cus = 0, clk_khz = 0;
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    CK(hipDeviceGetAttribute(&clk_khz, hipDeviceAttributeClockRate, 0));
    float* out = nullptr;
    CK(hipMalloc(&out, (size_t)cus * 512 * 4));
    const int iters = 20000;
    double tf[3], mhz[3];
    for (int k = 0; k < 3; ++k) {
        auto launch = [&] {
            if (k == 0) hipLaunchKernelGGL(mfma_kernel<0>, dim3(cus), dim3(512), 0, 0, out, iters);
            else if (k == 1) hipLaunchKernelGGL(mfma_kernel<1>, dim3(cus), dim3(512), 0, 0, out, iters);
            else hipLaunchKernelGGL(mfma_kernel<2>, dim3(cus), dim3(512), 0, 0, out, iters);
        };
        const float ms = time_ms(launch, 3);
        unsigned long long ticks[1];
        CK(hipMemcpyFromSymbol(ticks, HIP_SYMBOL(g_ticks), sizeof(ticks)));
        const double flop_per = k == 2 ? 2.0 * 32 * 32 * 64 : 2.0 * 32 * 32 * 16;
        const double flops = flop_per * 4.0 * iters * 8.0 * cus;   // 8 waves x 4 chains per CU
        tf[k] = flops / (ms * 1e-3) / 1e12;
        mhz[k] = (double)ticks[0] / (ms * 1e3);   // s_memtime ticks per microsecond of the launch
    }
    const size_t bytes = (size_t)2 << 30;
    uint4 *a = nullptr, *b = nullptr;
    CK(hipMalloc(&a, bytes));
    CK(hipMalloc(&b, bytes));
    CK(hipMemset(a, 1, bytes));
    const size_t n16 = bytes / 16;
    const float rms = time_ms([&] { hipLaunchKernelGGL(read_kernel, dim3(cus * 8), dim3(256), 0, 0, a, n16, b); }, 5);
    const float cms = time_ms([&] { hipLaunchKernelGGL(copy_kernel, dim3(cus * 8), dim3(256), 0, 0, a, b, n16); }, 5);
    printf("{\"cus\": %d, \"max_clock_mhz\": %d, \"bf16_32x32x16_tflops\": %.1f, \"f16_32x32x16_tflops\": %.1f, "
           "\"fp8_32x32x64_tflops\": %.1f, \"memtime_mhz_during_mfma\": [%.0f, %.0f, %.0f], "
           "\"hbm_read_gbps\": %.1f, \"hbm_copy_gbps\": %.1f}\n",
           cus, clk_khz / 1000, tf[0], tf[1], tf[2], mhz[0], mhz[1], mhz[2], bytes / (rms * 1e-3) / 1e9,
           2.0 * bytes / (cms * 1e-3) / 1e9);
    return 0;
}
