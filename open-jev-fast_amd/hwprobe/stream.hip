// Hardware probe (MI355X): the per-CU operand stream of a whole-M projection tile at M = 288, without compute.
// Each of the launch's workgroups (one per CU, 8 waves) streams
//   x: XR rows x K of an L2-resident activation (every workgroup reads the same rows), global -> LDS by DMA into a
//      ring of 3 stages of 64 k, one barrier per stage (MODE bit 0);
//   W: 128 weight rows x K from HBM straight into registers, D stages ahead (MODE bit 1), in one of two layouts:
//      LAYOUT 0 = the stage-major packed layout [K/64][N/16][16][64] (a k32 half of a 16 x 64 block is 16 rows x
//      64 B per instruction: half cache lines), LAYOUT 1 = 16 x 32 blocks of 1 KB (whole lines);
//   MODE bit 2: only waves 0-3 issue the x DMAs; bit 3: only waves 4-7 issue the W loads.
// The weights rotate over three 335 MB copies, so every W byte comes from HBM. Prints the time per launch.
// Build and run: hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops stream.hip \
//     -o /tmp/stream && /tmp/stream
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>

__device__ __forceinline__ __amdgpu_buffer_rsrc_t mk(const void* b, int64_t n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(b), (short)0, (int)(n > 0x7fffffff ? 0x7fffffff : n), 0x00020000);
}
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

template <int MODE, int LAYOUT, int D, int XR = 288>  // MODE bit0: x DMA, bit1: W loads
__global__ void __launch_bounds__(512) stream(const uint16_t* x, const uint16_t* w, int K, int N, float* out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int M = 288;
  const int nst = K / 64;
  const __amdgpu_buffer_rsrc_t rx = mk(x, (int64_t)M * K * 2), rw = mk(w, (int64_t)N * K * 2);
  // x DMA: 36 blocks of 8 rows x 128 B per stage; wave takes blocks wave, wave + 8, ...
  const int lrow = lane >> 3, lch = lane & 7;
  // W: fragment f = blockIdx.x * 8 + wave
  const bool xw = (MODE & 4) ? wave < 4 : true;          // waves that issue x DMAs
  const bool ww = (MODE & 8) ? wave >= 4 : true;         // waves that issue W loads
  const int f = (MODE & 8) ? blockIdx.x * 8 + (wave - 4) * 2 : blockIdx.x * 8 + wave;
  uint32_t wo0, wo1, wstep;
  if (LAYOUT == 0) {  // element (n, k) at ((k/64 * N/16 + n/16) * 16 + n%16) * 64 + k%64
    const uint32_t base = (uint32_t)(f * 16 + (lane & 15)) * 128u + (uint32_t)(lane >> 4) * 16u;
    wo0 = base; wo1 = base + 64; wstep = (uint32_t)N * 128u;  // per 64-k stage: N/16 blocks of 2 KB
  } else {  // element (n, k) at ((k/32 * N/16 + n/16) * 16 + n%16) * 32 + k%32
    const uint32_t base = (uint32_t)f * 1024u + (uint32_t)lane * 16u;
    wo0 = base; wo1 = base + (uint32_t)N * 64u; wstep = (uint32_t)N * 128u;
  }
  uint4 acc = {0, 0, 0, 0};
  (void)xw;
  uint4 ring[D][4];
  auto wload = [&](int s) {
    const uint32_t so = (uint32_t)s * wstep;
    const int slot = s % D;
    ring[slot][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo0 + so, 0, 2));
    ring[slot][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo1 + so, 0, 2));
    if (MODE & 8) {
      const uint32_t fo = LAYOUT == 0 ? 2048u : 1024u;
      ring[slot][2] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo0 + fo + so, 0, 2));
      ring[slot][3] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo1 + fo + so, 0, 2));
    }
  };
  auto xdma = [&](int s) {
    uint8_t* dst = smem + (s % 3) * (M * 128);
    const int nxw = (MODE & 4) ? 4 : 8;
    for (int b = wave; b < XR / 8; b += nxw) {
      const uint32_t vo = (uint32_t)((b * 8 + lrow) * K * 2 + lch * 16);
      dma16(rx, dst + b * 1024, vo, (uint32_t)s * 128u);
    }
  };
  if ((MODE & 1) && xw) { xdma(0); xdma(1); }
  if ((MODE & 2) && ww)
#pragma unroll
    for (int s = 0; s < D; ++s) wload(s);
  for (int s0 = 0; s0 < nst; s0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int s = s0 + j;
      if ((MODE & 2) && ww) {
        acc.x ^= ring[j][0].x ^ ring[j][1].y;
        acc.y ^= ring[j][0].z ^ ring[j][1].w;
        if (MODE & 8) acc.w ^= ring[j][2].x ^ ring[j][3].y;
        if (s + D < nst) wload(s + D);
      }
      if (MODE & 1) {
        if (xw && s + 2 < nst) xdma(s + 2);
        if (xw) {
          if ((MODE & 3) == 1 || (MODE & 8)) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
          else asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        }
        __builtin_amdgcn_s_barrier();
        const uint4 v = *reinterpret_cast<const uint4*>(smem + ((s + 1) % 3) * (M * 128) + (threadIdx.x * 16) % (M * 128));
        acc.z ^= v.x;
      }
    }
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x1234567u) out[blockIdx.x] = 1.f;
}

int main() {
  const int K = 5120, M = 288, N = 32768;
  uint16_t *x, *w[3]; float* out;
  hipMalloc(&x, (size_t)M * K * 2); hipMemset(x, 0, (size_t)M * K * 2);
  for (int i = 0; i < 3; ++i) { hipMalloc(&w[i], (size_t)N * K * 2); hipMemset(w[i], 0, (size_t)N * K * 2); }
  hipMalloc(&out, 4096);
  hipEvent_t a, b; hipEventCreate(&a); hipEventCreate(&b);
  auto run = [&](auto kern, const char* nm, int grid = 256) {
    hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 3 * M * 128);
    for (int i = 0; i < 6; ++i) hipLaunchKernelGGL(kern, dim3(grid), dim3(512), 3 * M * 128, 0, x, w[i % 3], K, N, out);
    hipDeviceSynchronize();
    hipEventRecord(a);
    for (int i = 0; i < 30; ++i) hipLaunchKernelGGL(kern, dim3(grid), dim3(512), 3 * M * 128, 0, x, w[i % 3], K, N, out);
    hipEventRecord(b); hipEventSynchronize(b);
    float ms; hipEventElapsedTime(&ms, a, b);
    const double us = ms * 1000 / 30;
    printf("%-36s grid %3d %8.2f us\n", nm, grid, us);
  };
  run(stream<1, 1, 4>, "x DMA only, 288 rows");
  run(stream<1, 1, 4, 144>, "x DMA only, 144 rows");
  run(stream<1, 1, 4, 72>, "x DMA only, 72 rows");
  run(stream<1, 1, 4>, "x DMA only, 288 rows", 128);
  run(stream<1, 1, 4>, "x DMA only, 288 rows", 32);
  run(stream<1, 1, 4>, "x DMA only, 288 rows", 8);
  run(stream<2, 1, 8>, "W only, whole lines, D8");
  run(stream<2, 0, 8>, "W only, half lines, D8");
  run(stream<3, 1, 8>, "x 288 + W whole lines");
  run(stream<3, 1, 8, 144>, "x 144 + W whole lines");
  run(stream<3, 1, 8, 72>, "x 72 + W whole lines");
  run(stream<3, 0, 8>, "x 288 + W half lines");
  run(stream<15, 1, 8>, "x by waves 0-3, W by waves 4-7");
  run(stream<7, 1, 8>, "x by waves 0-3, W by all");
  return 0;
}
