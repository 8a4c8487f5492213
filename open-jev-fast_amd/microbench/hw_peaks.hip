// Hardware ceilings of the MI355X this path is tuned for: bf16 MFMA issue rate (16x16x32 and 32x32x16) and the
// shader clock under MFMA load, streaming HBM read and copy bandwidth, and LDS ds_read_b128 bandwidth.
//
//   hipcc --offload-arch=gfx950 -O3 open-jev-fast_amd/microbench/hw_peaks.hip -o hw_peaks && ./hw_peaks
//
// These numbers, not the published peaks, say how close a kernel can get: the roofline fractions of the projection
// kernels are quoted against the published 8 TB/s and 2.5 PFLOP/s.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <vector>
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
#define CK(x) do{hipError_t e=(x); if(e){printf("err %s line %d\n",hipGetErrorString(e),__LINE__); return 1;}}while(0)

__global__ void mfma16(float* out, int iters, long long* clk) {
  bf16x8 a; for (int i=0;i<8;i++) a[i]=(__bf16)(threadIdx.x*0.001f+i);
  f32x4 c[8]; for(int j=0;j<8;j++) c[j]=f32x4{0,0,0,0};
  long long t0 = clock64(); long long w0 = wall_clock64();
  for (int it=0; it<iters; ++it) {
#pragma unroll
    for(int j=0;j<8;j++) c[j]=__builtin_amdgcn_mfma_f32_16x16x32_bf16(a,a,c[j],0,0,0);
  }
  long long t1 = clock64(); long long w1 = wall_clock64();
  float s=0; for(int j=0;j<8;j++) s+=c[j][0]+c[j][1]+c[j][2]+c[j][3];
  out[blockIdx.x*blockDim.x+threadIdx.x]=s;
  if (threadIdx.x==0 && blockIdx.x==0) { clk[0]=t1-t0; clk[1]=w1-w0; }
}
__global__ void mfma32(float* out, int iters) {
  bf16x8 a; for (int i=0;i<8;i++) a[i]=(__bf16)(threadIdx.x*0.001f+i);
  f32x16 c[4]; for(int j=0;j<4;j++) for(int e=0;e<16;e++) c[j][e]=0;
  for (int it=0; it<iters; ++it) {
#pragma unroll
    for(int j=0;j<4;j++) c[j]=__builtin_amdgcn_mfma_f32_32x32x16_bf16(a,a,c[j],0,0,0);
  }
  float s=0; for(int j=0;j<4;j++) s+=c[j][0]+c[j][5];
  out[blockIdx.x*blockDim.x+threadIdx.x]=s;
}
__global__ void readbw(const uint4* __restrict__ p, size_t n, uint4* out) {
  uint4 acc = make_uint4(0,0,0,0);
  for (size_t i = blockIdx.x*(size_t)blockDim.x+threadIdx.x; i<n; i+= (size_t)gridDim.x*blockDim.x) {
    uint4 v = p[i]; acc.x^=v.x; acc.y^=v.y; acc.z^=v.z; acc.w^=v.w; }
  if ((acc.x&0xffff)==0x1234) out[0]=acc;
}
__global__ void copybw(const uint4* __restrict__ p, uint4* __restrict__ q, size_t n) {
  for (size_t i = blockIdx.x*(size_t)blockDim.x+threadIdx.x; i<n; i+= (size_t)gridDim.x*blockDim.x) q[i]=p[i];
}
__global__ void ldsbw(float* out, int iters) {
  __shared__ uint4 s[4096];
  for (int i=threadIdx.x;i<4096;i+=blockDim.x) s[i]=make_uint4(i,i,i,i);
  __syncthreads();
  uint4 acc=make_uint4(0,0,0,0); int idx=threadIdx.x;
  for (int it=0; it<iters; ++it) {
#pragma unroll
    for (int j=0;j<8;j++){ uint4 v=s[(idx + j*64)&4095]; acc.x+=v.x; acc.y^=v.y; }
    idx += 7;
  }
  out[blockIdx.x*blockDim.x+threadIdx.x]=acc.x+acc.y;
}
int main() {
  hipDeviceProp_t pr; CK(hipGetDeviceProperties(&pr,0));
  printf("device %s CUs %d clock %d kHz memclk %d kHz bus %d l2 %d\n", pr.name, pr.multiProcessorCount, pr.clockRate, pr.memoryClockRate, pr.memoryBusWidth, pr.l2CacheSize);
  float* out; CK(hipMalloc(&out, 64<<20)); long long* clk; CK(hipMalloc(&clk, 64));
  hipEvent_t a,b; hipEventCreate(&a); hipEventCreate(&b); float ms;
  for (int wpb : {4, 8, 16}) {
    int blocks = 256*2, iters=2000;
    hipLaunchKernelGGL(mfma16, dim3(blocks), dim3(64*wpb), 0, 0, out, 10, clk);
    hipEventRecord(a); hipLaunchKernelGGL(mfma16, dim3(blocks), dim3(64*wpb), 0, 0, out, iters, clk); hipEventRecord(b); hipEventSynchronize(b);
    hipEventElapsedTime(&ms,a,b); long long c[2]; hipMemcpy(c, clk, 16, hipMemcpyDeviceToHost);
    double fl = 2.0*16*16*32*8*(double)iters*blocks*wpb;
    printf("mfma16x16x32 waves/blk %d: %.3f ms  %.1f TFLOP/s  cycles/mfma(wave0) %.2f  clk64/wall %.3f (wall 100MHz)\n", wpb, ms, fl/ms/1e9, (double)c[0]/(iters*8), (double)c[0]/c[1]);
  }
  for (int wpb : {4, 8}) {
    int blocks = 512, iters=2000;
    hipLaunchKernelGGL(mfma32, dim3(blocks), dim3(64*wpb), 0, 0, out, 10);
    hipEventRecord(a); hipLaunchKernelGGL(mfma32, dim3(blocks), dim3(64*wpb), 0, 0, out, iters); hipEventRecord(b); hipEventSynchronize(b);
    hipEventElapsedTime(&ms,a,b);
    double fl = 2.0*32*32*16*4*(double)iters*blocks*wpb;
    printf("mfma32x32x16 waves/blk %d: %.3f ms  %.1f TFLOP/s\n", wpb, ms, fl/ms/1e9);
  }
  size_t bytes = 2ull<<30; uint4 *p,*q; CK(hipMalloc(&p, bytes)); CK(hipMalloc(&q, bytes)); hipMemset(p, 1, bytes); hipMemset(q,0,bytes);
  size_t n = bytes/16;
  for (int g : {1024, 2048, 4096, 8192}) {
    hipLaunchKernelGGL(readbw, dim3(g), dim3(256), 0, 0, p, n, (uint4*)out);
    hipEventRecord(a); for(int r=0;r<5;r++) hipLaunchKernelGGL(readbw, dim3(g), dim3(256), 0, 0, p, n, (uint4*)out); hipEventRecord(b); hipEventSynchronize(b);
    hipEventElapsedTime(&ms,a,b); printf("read %zu MB grid %d: %.1f GB/s\n", bytes>>20, g, 5*bytes/ms/1e6);
  }
  for (int g : {2048, 8192}) {
    hipLaunchKernelGGL(copybw, dim3(g), dim3(256), 0, 0, p, q, n);
    hipEventRecord(a); for(int r=0;r<5;r++) hipLaunchKernelGGL(copybw, dim3(g), dim3(256), 0, 0, p, q, n); hipEventRecord(b); hipEventSynchronize(b);
    hipEventElapsedTime(&ms,a,b); printf("copy %zu MB grid %d: %.1f GB/s (r+w)\n", bytes>>20, g, 5*2.0*bytes/ms/1e6);
  }
  {
    int blocks=1024, iters=4000;
    hipLaunchKernelGGL(ldsbw, dim3(blocks), dim3(256), 0, 0, out, 10);
    hipEventRecord(a); hipLaunchKernelGGL(ldsbw, dim3(blocks), dim3(256), 0, 0, out, iters); hipEventRecord(b); hipEventSynchronize(b);
    hipEventElapsedTime(&ms,a,b);
    double by = 16.0*8*iters*blocks*256;
    printf("lds read b128: %.1f TB/s total, %.1f B/clk/CU at 2.4GHz\n", by/ms/1e9, by/ms/1e-3/256/2.4e9);
  }
  return 0;
}
