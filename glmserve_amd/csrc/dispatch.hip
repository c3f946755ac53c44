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

int launch_dispatch(const int* ids, int n, int topk, int E, int* offsets, int* sorted_tok,
                    int* sorted_slot, int* inv, int* tiles, int* ntiles, int tile_rows,
                    int with_shared, int mode, hipStream_t s) {
    if (E > kDispMaxE || E < 1) return -2;
    const DispOut d{offsets, sorted_tok, sorted_slot, inv, reinterpret_cast<int4*>(tiles),
                    ntiles, tile_rows, with_shared, mode};
    hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(kDispThreads), 0, s, ids, n, topk, E, d);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // namespace glmmoe
