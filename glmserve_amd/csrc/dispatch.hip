// Stand-alone dispatch kernel (the body is in dispatch.hpp).
//
// Reference: cuda/moe_dispatch.cu:16-45, cuda/qgemm.cu:966-989.
#include "dispatch.hpp"
#include "kernels.hpp"

namespace glmmoe {

constexpr int kDispThreads = 1024;

__global__ __launch_bounds__(kDispThreads) void dispatch_kernel(const int* __restrict__ ids,
                                                                int n, int topk, int E,
                                                                DispOut d) {
    __shared__ int lds[dispatch_lds_ints<kDispThreads>()];
    dispatch_block<kDispThreads>(ids, n, topk, E, d, lds);
}

// Large batches: chunk histograms, then every chunk permutes its own ids
// (bases from all the histograms), in parallel.
constexpr int kDispChunk = 2048;          // ids per workgroup
// Total ids from which the multi-workgroup path runs. Measured per dispatch:
// 7200 ids 29.5 -> 20.1 us, 4160 ids 21.0 -> 18.8 us; at 2400 ids the single
// workgroup is faster (15.9 against 18.2 us).
constexpr int kDispMultiMin = 4096;
constexpr int kDispMaxChunks = 256;

__global__ __launch_bounds__(kDispThreads) void dispatch_count_kernel(const int* __restrict__ ids,
                                                                      int total, int E,
                                                                      int* __restrict__ bcounts) {
    __shared__ int cnt[kDispMaxE];
    const int b = blockIdx.x, tid = threadIdx.x;
    for (int e = tid; e < E; e += kDispThreads) cnt[e] = 0;
    __syncthreads();
    const int i0 = b * kDispChunk, i1 = min(total, i0 + kDispChunk);
    for (int i = i0 + tid; i < i1; i += kDispThreads) {
        const int e = ids[i];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    for (int e = tid; e < E; e += kDispThreads) bcounts[(size_t)b * E + e] = cnt[e];
}

__global__ __launch_bounds__(kDispThreads) void dispatch_chunk_kernel(const int* __restrict__ ids,
                                                                      int n, int topk, int E,
                                                                      DispOut d,
                                                                      const int* __restrict__ bcounts) {
    __shared__ int lds[dispatch_lds_ints<kDispThreads>()];
    const int total = n * topk;
    const int b = blockIdx.x, i0 = b * kDispChunk, i1 = min(total, i0 + kDispChunk);
    dispatch_block<kDispThreads>(ids, n, topk, E, d, lds, i0, i1, bcounts, (int)gridDim.x, b);
}

size_t dispatch_scratch_bytes(int n, int topk, int E) {
    const long total = (long)n * topk;
    if (total < kDispMultiMin) return 0;
    return (size_t)((total + kDispChunk - 1) / kDispChunk) * E * 4;
}

int launch_dispatch(const int* ids, int n, int topk, int E, int* offsets, int* sorted_tok,
                    int* sorted_slot, int* inv, int* tiles, int* ntiles, int tile_rows,
                    int with_shared, int mode, hipStream_t s, int* scratch, int half_rows,
                    unsigned int* zero, int nzero) {
    if (E > kDispMaxE || E < 1) return -2;
    const DispOut d{offsets, sorted_tok, sorted_slot, inv, reinterpret_cast<int4*>(tiles),
                    ntiles, tile_rows, with_shared, mode, half_rows, zero, nzero};
    const long total = (long)n * topk;
    const long nblk = (total + kDispChunk - 1) / kDispChunk;
    if (scratch && total >= kDispMultiMin && nblk <= kDispMaxChunks) {
        hipLaunchKernelGGL(dispatch_count_kernel, dim3((unsigned)nblk), dim3(kDispThreads), 0, s,
                           ids, (int)total, E, scratch);
        if (hipGetLastError() != hipSuccess) return -4;
        hipLaunchKernelGGL(dispatch_chunk_kernel, dim3((unsigned)nblk), dim3(kDispThreads), 0, s,
                           ids, n, topk, E, d, scratch);
        return hipGetLastError() == hipSuccess ? 0 : -4;
    }
    hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(kDispThreads), 0, s, ids, n, topk, E, d);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace glmmoe
