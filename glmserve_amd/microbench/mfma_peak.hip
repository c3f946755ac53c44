// MFMA throughput probe for gfx950: back-to-back independent accumulation
// chains of v_mfma_f32_16x16x32_bf16 and v_mfma_f32_32x32x16_bf16, one or two
// 256-thread workgroups per CU. Prints TFLOP/s and cycles per MFMA per SIMD.
// Build and run (GPU box):
//   hipcc --offload-arch=gfx950 -O3 glmserve_amd/microbench/mfma_peak.hip -o /tmp/mfma_peak
//   /tmp/mfma_peak
#include <hip/hip_runtime.h>
#include <cstdio>
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
__global__ __launch_bounds__(256) void k16(float* out, int iters){
  bf16x8 a; bf16x8 b; for(int i=0;i<8;i++){a[i]=(__bf16)(threadIdx.x*0.001f+i); b[i]=(__bf16)(i*0.5f);}
  f4 c[8]; for(int j=0;j<8;j++) c[j]=f4{0,0,0,0};
  for(int it=0; it<iters; ++it){
#pragma unroll
    for(int j=0;j<8;j++) c[j]=__builtin_amdgcn_mfma_f32_16x16x32_bf16(a,b,c[j],0,0,0);
  }
  float s=0; for(int j=0;j<8;j++) s+=c[j][0]+c[j][3]; out[blockIdx.x*256+threadIdx.x]=s;
}
__global__ __launch_bounds__(256) void k32(float* out, int iters){
  bf16x8 a; bf16x8 b; for(int i=0;i<8;i++){a[i]=(__bf16)(threadIdx.x*0.001f+i); b[i]=(__bf16)(i*0.5f);}
  f16v c[4]; for(int j=0;j<4;j++) for(int e=0;e<16;e++) c[j][e]=0;
  for(int it=0; it<iters; ++it){
#pragma unroll
    for(int j=0;j<4;j++) c[j]=__builtin_amdgcn_mfma_f32_32x32x16_bf16(a,b,c[j],0,0,0);
  }
  float s=0; for(int j=0;j<4;j++) s+=c[j][0]+c[j][15]; out[blockIdx.x*256+threadIdx.x]=s;
}
int main(){
  float* o; (void)hipMalloc(&o, 256*1024*8*sizeof(float));
  int cus; hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0);
  int clk; hipDeviceGetAttribute(&clk, hipDeviceAttributeClockRate, 0);
  hipEvent_t e0,e1; hipEventCreate(&e0); hipEventCreate(&e1);
  int iters=20000; 
  for (int occ : {1,2}) {
    int blocks = cus*occ;
    hipLaunchKernelGGL(k16, dim3(blocks), dim3(256),0,0,o,100); hipDeviceSynchronize();
    hipEventRecord(e0); hipLaunchKernelGGL(k16, dim3(blocks), dim3(256),0,0,o,iters); hipEventRecord(e1); hipEventSynchronize(e1);
    float ms; hipEventElapsedTime(&ms,e0,e1);
    double fl = 2.0*16*16*32*8.0*iters*blocks*4;
    printf("16x16x32 bf16 occ=%d: %.1f TFLOP/s  (cycles/mfma/SIMD at %d MHz: %.1f)\n", occ, fl/ms/1e9, clk/1000, ms*1e-3*clk*1e3/(8.0*iters*occ));
    hipLaunchKernelGGL(k32, dim3(blocks), dim3(256),0,0,o,100); hipDeviceSynchronize();
    hipEventRecord(e0); hipLaunchKernelGGL(k32, dim3(blocks), dim3(256),0,0,o,iters); hipEventRecord(e1); hipEventSynchronize(e1);
    hipEventElapsedTime(&ms,e0,e1);
    fl = 2.0*32*32*16*4.0*iters*blocks*4;
    printf("32x32x16 bf16 occ=%d: %.1f TFLOP/s  (cycles/mfma/SIMD: %.1f)\n", occ, fl/ms/1e9, ms*1e-3*clk*1e3/(4.0*iters*occ));
  }
  printf("CUs=%d clock=%d kHz\n", cus, clk);
  return 0;
}
