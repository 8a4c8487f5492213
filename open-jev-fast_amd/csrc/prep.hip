// Full-attention prep: the consumer of the full-attention layers' in-projection output.
//
// Reference: fullattn_prep2_k (src/kernels.cu:302-355), called from forward_gtree as
// K.fullattn_prep2(proj, qw1, kw1, cos, sin, 1, N, HQ, HKV, D, eps) (src/fastmodel.py:462). proj [N, P] bf16 with
// P = HQ 2D + 2 HKV D; per token n and head:
//   q head h: x = proj[n][2hD .. 2hD+D), gate head h = proj[n][2hD+D .. 2hD+2D);
//   k head h: x = proj[n][2 HQ D + hD ..); v head h = proj[n][2 HQ D + HKV D + hD ..).
//   q and k: xn = bf16((x * rsqrt(sum x^2 / D + eps)) * w1[d]) with w1 = qw1 / kw1 [D] fp32, then on the first RD
//   dims the rotate-half RoPE: out = bf16(bf16(xn * cos[n][d]) + bf16(rh * sin[n][d])), rh = -xn[d + RD/2] for
//   d < RD/2 and xn[d - RD/2] for RD/2 <= d < RD; dims >= RD keep xn.
//   Outputs (B = 1, T = N): qt [HQ, N, D], kt [HKV, N, D], vt [HKV, N, D] (head-major for attention) and
//   gate [N, HQ D].
//
// One wave64 per (token, head task), 4 consecutive dims per lane (D = 256): the row's sum of squares is a wave
// butterfly, and the RoPE partner of lane l is lane l ^ (RD / 8), because dims d and d +- RD/2 sit RD/8 lanes
// apart and RD/8 is a power of two below 16 (RD in {32, 64, 128}).
#include "ojx_internal.h"

namespace ojx {

namespace {

__device__ __forceinline__ void unpack4(uint2 a, float (&v)[4]) {
  v[0] = bf2f(a.x & 0xffffu); v[1] = bf2f(a.x >> 16); v[2] = bf2f(a.y & 0xffffu); v[3] = bf2f(a.y >> 16);
}
__device__ __forceinline__ uint2 pack4(const float (&v)[4]) { return make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3])); }

}  // namespace

// FD: dims per lane (D / 64)
__global__ void __launch_bounds__(256) fullattn_prep_k(const uint16_t* __restrict__ proj, int64_t N, int HQ, int HKV,
                                                       int RD, float eps, const float* __restrict__ qw1,
                                                       const float* __restrict__ kw1, const uint16_t* __restrict__ cosb,
                                                       const uint16_t* __restrict__ sinb, uint16_t* __restrict__ qt,
                                                       uint16_t* __restrict__ kt, uint16_t* __restrict__ vt,
                                                       uint16_t* __restrict__ gate) {
  constexpr int D = 256;
  const int lane = threadIdx.x & 63;
  const int ntask = HQ + 2 * HKV;
  const int64_t wid = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (wid >= N * ntask) return;
  const int64_t n = wid / ntask;
  const int task = (int)(wid - n * ntask);
  const int64_t P = (int64_t)(2 * HQ + 2 * HKV) * D;
  const uint16_t* row = proj + n * P;
  const int d0 = lane * 4;
  if (task >= HQ + HKV) {  // v head: a copy into [HKV, N, D]
    const int h = task - HQ - HKV;
    *reinterpret_cast<uint2*>(vt + ((int64_t)h * N + n) * D + d0) =
        *reinterpret_cast<const uint2*>(row + 2 * HQ * D + HKV * D + h * D + d0);
    return;
  }
  const bool isq = task < HQ;
  const int h = isq ? task : task - HQ;
  if (isq)  // gate head: a copy into [N, HQ D]
    *reinterpret_cast<uint2*>(gate + n * (int64_t)(HQ * D) + h * D + d0) =
        *reinterpret_cast<const uint2*>(row + (int64_t)h * 2 * D + D + d0);
  float x[4];
  unpack4(*reinterpret_cast<const uint2*>(row + (isq ? (int64_t)h * 2 * D : 2 * HQ * D + (int64_t)h * D) + d0), x);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) ss += x[j] * x[j];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float r = rsqrtf(ss / (float)D + eps);
  const float* w1 = isq ? qw1 : kw1;
  const float4 wv = *reinterpret_cast<const float4*>(w1 + d0);
  float nv[4] = {rbf((x[0] * r) * wv.x), rbf((x[1] * r) * wv.y), rbf((x[2] * r) * wv.z), rbf((x[3] * r) * wv.w)};
  const int hl = RD >> 3;  // partner lane distance
  float pv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) pv[j] = __shfl_xor(nv[j], hl);
  float out[4];
  if (d0 < RD) {
    float c[4], s[4];
    unpack4(*reinterpret_cast<const uint2*>(cosb + n * RD + d0), c);
    unpack4(*reinterpret_cast<const uint2*>(sinb + n * RD + d0), s);
    const bool lo = d0 < RD / 2;
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = rbf(rbf(nv[j] * c[j]) + rbf((lo ? -pv[j] : pv[j]) * s[j]));
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = nv[j];
  }
  uint16_t* dst = isq ? qt : kt;
  *reinterpret_cast<uint2*>(dst + ((int64_t)h * N + n) * D + d0) = pack4(out);
}

hipError_t launch_fullattn_prep(const uint16_t* proj, int64_t N, int HQ, int HKV, int RD, float eps,
                                const float* qw1, const float* kw1, const uint16_t* cosb, const uint16_t* sinb,
                                uint16_t* qt, uint16_t* kt, uint16_t* vt, uint16_t* gate, hipStream_t st) {
  const int64_t waves = N * (HQ + 2 * HKV);
  hipLaunchKernelGGL(fullattn_prep_k, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, proj, N, HQ, HKV, RD, eps,
                     qw1, kw1, cosb, sinb, qt, kt, vt, gate);
  return hipGetLastError();
}

}  // namespace ojx
