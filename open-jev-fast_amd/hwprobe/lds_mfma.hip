// Hardware probe (MI355X): LDS read bandwidth per CU, and the bf16 16x16x32 MFMA rate when each wave also reads R
// 1 KB fragments from LDS per F MFMAs (the operand traffic of a GEMM tile whose waves own F / R W fragments per x
// fragment read). Constant operand data. One workgroup per CU.
// Build and run: hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops lds_mfma.hip \
//     -o /tmp/lds_mfma && /tmp/lds_mfma
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// R ds_read_b128 + F MFMAs per iteration per wave; acc over F/R... each read feeds F/R MFMAs
template <int R, int F, int NACC>
__global__ void __launch_bounds__(512) mix(float* out, int iters) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[64 * 1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < 64 * 1024 / 4; i += blockDim.x) reinterpret_cast<float*>(lds)[i] = 0.001f * (i & 7);
  __syncthreads();
  f32x4 acc[NACC];
  for (int i = 0; i < NACC; ++i) acc[i] = f32x4{0, 0, 0, 0};
  bf16x8 a = *reinterpret_cast<const bf16x8*>(lds + lane * 16);
  uint32_t base = (wave * 4096 + lane * 16) & 0xffff;
  for (int it = 0; it < iters; ++it) {
    bf16x8 b[R > 0 ? R : 1];
#pragma unroll
    for (int r = 0; r < R; ++r) b[r] = *reinterpret_cast<const bf16x8*>(lds + ((base + r * 1024 + it * 64) & 0xfff0));
#pragma unroll
    for (int f = 0; f < F; ++f) {
      const bf16x8 bb = R > 0 ? b[f % (R > 0 ? R : 1)] : a;
      acc[f % NACC] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bb, acc[f % NACC], 0, 0, 0);
    }
  }
  float s = 0;
  for (int i = 0; i < NACC; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  if (s == 1234.5f) out[blockIdx.x] = s;
}

// pure LDS read bandwidth: each wave reads 1 KB per ds_read_b128 instruction
template <int U>
__global__ void __launch_bounds__(1024) ldsbw(float* out, int iters) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[64 * 1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < 64 * 1024 / 4; i += blockDim.x) reinterpret_cast<float*>(lds)[i] = (float)(i & 7);
  __syncthreads();
  uint4 x = {0, 0, 0, 0};
  uint32_t base = (wave * 2048 + lane * 16);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint4 v = *reinterpret_cast<const uint4*>(lds + ((base + u * 1024 + it * 16) & 0xfff0));
      x.x ^= v.x; x.y ^= v.y; x.z ^= v.z; x.w ^= v.w;
    }
  }
  if ((x.x ^ x.y ^ x.z ^ x.w) == 0x12345) out[blockIdx.x] = 1;
}

int main() {
  float* out; hipMalloc(&out, 1 << 20);
  hipEvent_t a, b; hipEventCreate(&a); hipEventCreate(&b);
  int dev; hipGetDevice(&dev); hipDeviceProp_t pr; hipGetDeviceProperties(&pr, dev);
  printf("CUs %d clock %d kHz\n", pr.multiProcessorCount, pr.clockRate);
  auto time = [&](auto launch, int reps) {
    launch(); hipDeviceSynchronize();
    hipEventRecord(a); for (int i = 0; i < reps; ++i) launch(); hipEventRecord(b); hipEventSynchronize(b);
    float ms; hipEventElapsedTime(&ms, a, b); return ms / reps * 1e-3;
  };
  const int CUS = 256;
  for (int thr : {256, 512, 1024}) {
    int iters = 4000;
    double t = time([&] { hipLaunchKernelGGL(ldsbw<8>, dim3(CUS), dim3(thr), 0, 0, out, iters); }, 5);
    double bytes = (double)CUS * (thr / 64) * iters * 8 * 1024;
    printf("LDS read  %4d thr/WG: %.2f TB/s total, %.1f B/clk/CU at 2.1 GHz\n", thr, bytes / t / 1e12,
           bytes / t / CUS / 2.1e9);
  }
  // MFMA with LDS reads: flops per MFMA 16384
  auto mixrun = [&](auto kern, const char* nm, int R, int F, int thr) {
    int iters = 2000;
    double t = time([&] { hipLaunchKernelGGL(kern, dim3(CUS), dim3(thr), 0, 0, out, iters); }, 5);
    double fl = (double)CUS * (thr / 64) * iters * F * 16384.0;
    double by = (double)CUS * (thr / 64) * iters * R * 1024.0;
    printf("%-28s thr %3d: %.3f PFLOP/s  LDS %.1f B/clk/CU\n", nm, thr, fl / t / 1e15, by / t / CUS / 2.1e9);
  };
  mixrun(mix<0, 32, 16>, "mfma only", 0, 32, 256);
  mixrun(mix<0, 32, 16>, "mfma only", 0, 32, 512);
  mixrun(mix<18, 36, 36>, "R18 F36 (W-direct 32 rows)", 18, 36, 512);
  mixrun(mix<18, 36, 36>, "R18 F36", 18, 36, 256);
  mixrun(mix<14, 41, 41>, "R14 F41 (kx 144x288)", 14, 41, 512);
  mixrun(mix<18, 54, 54>, "R18 F54 (48 rows)", 18, 54, 512);
  mixrun(mix<9, 36, 36>, "R9 F36", 9, 36, 512);
  mixrun(mix<18, 18, 18>, "R18 F18", 18, 18, 512);
  return 0;
}
