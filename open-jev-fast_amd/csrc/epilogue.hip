// Second-pass and standalone epilogue kernels of the projection path (HBM-bound row / elementwise work).
//
//   reduce_bf16_k     y = bf16(sum_s parts[s])                                   (split-K plain projection)
//   reduce_silu_k     out = bf16(bf16(silu(bf16 g)) * bf16 u), g/u = sum_s parts  (split-K gate-up)
//   add_rmsnorm_k     h = bf16(x + bf16(delta)); hn = bf16((h * rsqrt(mean h^2 + eps)) * w1), 0 where rowmask == 0
//                     delta = nothing | bf16 [M,H] | sum_s fp32 parts[s]
//                     (reference: add_rmsnorm_k src/kernels.cu:41-73, add_rmsnorm_sk2_k src/kernels.cu:1444-1501)
//   silu_mul_k        gu = [gate | up] row stride 2I -> out = bf16(bf16(silu(g)) * u), optionally through the
//                     65536-entry table (reference: silu_mul_k src/kernels.cu:76-89, silu_mul_lut_k :1304-1331)
//   act_tables_k      silu_b[bits] = bf16(silu(x)), sig_f[bits] = sigmoid(x) (reference: src/kernels.cu:1288-1301)
//   pack_gate_up_k    W_gu rows in blocks of 8: gate rows 4b..4b+3 then up rows 4b..4b+3 (the GEMM's fused
//                     SiLU.mul layout; the reference concatenates [gate; up], src/fastmodel.py:90)
//
// All loads and stores are 16-byte vectors; split partial planes are summed in ascending split order, the order
// of add_rmsnorm_sk2_k (src/kernels.cu:1464-1468), so results do not depend on the launch.
#include "ojx_internal.h"

namespace ojx {


// a[v] = sum over the S planes of the float4 at src + 4 v, added in ascending plane order. The loads go out eight
// planes at a time (indices clamped, extra planes not added) so that S planes cost about S/8 memory latencies
// rather than S: the reduction runs on few workgroups at small M, where latency is all there is.
template <int V>
__device__ __forceinline__ void sum_planes(const float* src, int S, int64_t ps, float4 (&a)[V]) {
#pragma unroll
  for (int v = 0; v < V; ++v) a[v] = *reinterpret_cast<const float4*>(src + 4 * v);
  for (int s0 = 1; s0 < S; s0 += 8) {
    float4 c[8][V];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t s = s0 + u < S ? s0 + u : S - 1;
#pragma unroll
      for (int v = 0; v < V; ++v) c[u][v] = *reinterpret_cast<const float4*>(src + s * ps + 4 * v);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const bool on = s0 + u < S;  // a select, not a branch: the loads above stay one batch
#pragma unroll
      for (int v = 0; v < V; ++v) {
        a[v].x = on ? a[v].x + c[u][v].x : a[v].x;
        a[v].y = on ? a[v].y + c[u][v].y : a[v].y;
        a[v].z = on ? a[v].z + c[u][v].z : a[v].z;
        a[v].w = on ? a[v].w + c[u][v].w : a[v].w;
      }
    }
  }
}

__global__ void __launch_bounds__(256) reduce_bf16_k(const float* __restrict__ parts, int S, int64_t ps,
                                                     uint16_t* __restrict__ y, int64_t ldy, int M, int N) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int n4 = N >> 2;
  if (idx >= (int64_t)M * n4) return;
  const int m = (int)(idx / n4), n = (int)(idx - (int64_t)m * n4) * 4;
  const float* src = parts + (int64_t)m * N + n;
  float4 sv[1];
  sum_planes<1>(src, S, ps, sv);
  const float4 s = sv[0];
  *reinterpret_cast<uint2*>(y + (int64_t)m * ldy + n) = make_uint2(pack2(s.x, s.y), pack2(s.z, s.w));
}

// parts: [S, M, N] with N = 2I packed as blocks of 8 (4 gate, 4 up); out: [M, I] row stride ldo.
__global__ void __launch_bounds__(256) reduce_silu_k(const float* __restrict__ parts, int S, int64_t ps,
                                                     uint16_t* __restrict__ out, int64_t ldo, int M, int N) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int nb = N >> 3;  // blocks of 8 packed columns = groups of 4 output columns
  if (idx >= (int64_t)M * nb) return;
  const int m = (int)(idx / nb), blk = (int)(idx - (int64_t)m * nb);
  const float* src = parts + (int64_t)m * N + blk * 8;
  float4 gu[2];
  sum_planes<2>(src, S, ps, gu);
  const float4 g = gu[0], u = gu[1];
  const float o0 = rbf(silu_f(rbf(g.x))) * rbf(u.x), o1 = rbf(silu_f(rbf(g.y))) * rbf(u.y);
  const float o2 = rbf(silu_f(rbf(g.z))) * rbf(u.z), o3 = rbf(silu_f(rbf(g.w))) * rbf(u.w);
  *reinterpret_cast<uint2*>(out + (int64_t)m * ldo + blk * 4) = make_uint2(pack2(o0, o1), pack2(o2, o3));
}

// One workgroup per row, H/8 threads, 8 contiguous elements per thread.
// MODE 0: h = x (no add); 1: h = bf16(x + delta); 2: h = bf16(x + bf16(sum of the S fp32 planes)). HN: write hn.
// Both are template parameters so that each variant is straight-line code and its loads (planes, x, w1) go out
// together; the split-K variant runs on one workgroup per row, where memory latency is most of its time.
template <int MODE, bool HN>
__global__ void __launch_bounds__(1024) add_rmsnorm_k(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ delta,
                                                      const float* __restrict__ parts, int S, int64_t ps,
                                                      const float* __restrict__ w1,
                                                      const int32_t* __restrict__ rowmask, float eps,
                                                      uint16_t* __restrict__ h_out, uint16_t* __restrict__ hn_out,
                                                      int H) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const int i = threadIdx.x * 8;
  float d[8];
  if constexpr (MODE == 2) {
    float4 ab[2];
    sum_planes<2>(parts + row * H + i, S, ps, ab);
    d[0] = rbf(ab[0].x); d[1] = rbf(ab[0].y); d[2] = rbf(ab[0].z); d[3] = rbf(ab[0].w);
    d[4] = rbf(ab[1].x); d[5] = rbf(ab[1].y); d[6] = rbf(ab[1].z); d[7] = rbf(ab[1].w);
  } else if constexpr (MODE == 1) {
    const uint4 da = *reinterpret_cast<const uint4*>(delta + row * H + i);
    const uint32_t dw[4] = {da.x, da.y, da.z, da.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) { d[2 * j] = bf2f(dw[j] & 0xffffu); d[2 * j + 1] = bf2f(dw[j] >> 16); }
  }
  const uint4 xa = *reinterpret_cast<const uint4*>(x + row * H + i);
  float4 wa = make_float4(0.f, 0.f, 0.f, 0.f), wb = wa;
  if constexpr (HN) {
    wa = *reinterpret_cast<const float4*>(w1 + i);
    wb = *reinterpret_cast<const float4*>(w1 + i + 4);
  }
  const uint32_t xw[4] = {xa.x, xa.y, xa.z, xa.w};
  float v[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) { v[2 * j] = bf2f(xw[j] & 0xffffu); v[2 * j + 1] = bf2f(xw[j] >> 16); }
  if constexpr (MODE != 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = rbf(v[j] + d[j]);
    *reinterpret_cast<uint4*>(h_out + row * H + i) =
        make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
  }
  if constexpr (HN) rmsnorm_row8(v, wa, wb, rowmask == nullptr || rowmask[row] != 0, eps, H, red, hn_out + row * H + i);
}

__global__ void __launch_bounds__(256) silu_mul_k(const uint16_t* __restrict__ gu, const uint16_t* __restrict__ tab,
                                                  uint16_t* __restrict__ out, int I, int64_t total8) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total8) return;
  const int64_t e = idx * 8;
  const int64_t row = e / I, col = e - row * I;
  const uint4 ga = *reinterpret_cast<const uint4*>(gu + row * 2 * I + col);
  const uint4 ua = *reinterpret_cast<const uint4*>(gu + row * 2 * I + I + col);
  const uint32_t gw[4] = {ga.x, ga.y, ga.z, ga.w}, uw[4] = {ua.x, ua.y, ua.z, ua.w};
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t gb = (j & 1) ? (gw[j >> 1] >> 16) : (gw[j >> 1] & 0xffffu);
    const uint32_t ub = (j & 1) ? (uw[j >> 1] >> 16) : (uw[j >> 1] & 0xffffu);
    const float s = tab != nullptr ? bf2f(tab[gb]) : rbf(silu_f(bf2f(gb)));
    o[j] = s * bf2f(ub);
  }
  *reinterpret_cast<uint4*>(out + e) =
      make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
}

__global__ void __launch_bounds__(256) act_tables_k(uint16_t* __restrict__ silu_b, float* __restrict__ sig_f) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 65536) return;
  const float x = bf2f((uint32_t)i);
  silu_b[i] = (uint16_t)f2bf(silu_f(x));
  sig_f[i] = sigmoid_f(x);
}

// packed row p: block b = p / 8, w = p % 8 -> gate row 4b + w (w < 4) or up row 4b + w - 4
__global__ void __launch_bounds__(256) pack_gate_up_k(const uint16_t* __restrict__ gate,
                                                      const uint16_t* __restrict__ up,
                                                      uint16_t* __restrict__ packed, int I, int K) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int cpr = K >> 3;
  if (idx >= (int64_t)2 * I * cpr) return;
  const int64_t p = idx / cpr;
  const int c = (int)(idx - p * cpr) * 8;
  const int64_t blk = p >> 3, w = p & 7;
  const uint16_t* src = (w < 4 ? gate : up) + (blk * 4 + (w & 3)) * K + c;
  *reinterpret_cast<uint4*>(packed + p * K + c) = *reinterpret_cast<const uint4*>(src);
}

// W row n, 8 columns k .. k+7 (k % 8 == 0) -> the packed layout: stage s = k / 64, row block nb = n / 16, offset
// ((s * N / 16 + nb) * 16 + n % 16) * 64 + k % 64. One thread per 16 bytes; reads and writes are both contiguous
// runs (a row's 128 bytes of one stage land in one 128-byte line of the packed buffer).
__global__ void __launch_bounds__(256) pack_weight_k(const uint16_t* __restrict__ w, uint16_t* __restrict__ wp,
                                                     int64_t N, int64_t K) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t cpr = K >> 3;
  if (idx >= N * cpr) return;
  const int64_t n = idx / cpr, k = (idx - n * cpr) * 8;
  const int64_t dst = (((k >> 6) * (N >> 4) + (n >> 4)) * 16 + (n & 15)) * 64 + (k & 63);
  *reinterpret_cast<uint4*>(wp + dst) = *reinterpret_cast<const uint4*>(w + n * K + k);
}

// The reference's split-K weight copy wsk [S, K/S, N] (src/fastmodel.py:186-188: wsk[s][k][n] = W[n][s K/S + k]) is
// W^T [K, N] row-major once its first two dims are merged; back to W [N, K]: a transpose through LDS. One workgroup
// per 64 x 64 block: 256 threads read 64 rows of 64 n (16 B each, two passes), then each writes 8 consecutive k of
// one n (16 B), so both global sides are 128-byte row pieces. The LDS row pitch of 72 elements puts the 8 rows a
// thread gathers on different banks. K and N are multiples of 8 (whole 16-byte pieces; partial blocks are guarded).
__global__ void __launch_bounds__(256) unsplit_weight_k(const uint16_t* __restrict__ wt, uint16_t* __restrict__ w,
                                                        int64_t K, int64_t N) {
  __shared__ uint16_t t[64][72];
  const int tid = threadIdx.x;
  const int64_t k0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int r = pass * 32 + (tid >> 3), c = (tid & 7) * 8;  // row k0 + r, columns n0 + c .. + 7
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (k0 + r < K && n0 + c < N) v = *reinterpret_cast<const uint4*>(wt + (k0 + r) * N + n0 + c);
    const uint32_t e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      t[r][c + 2 * j] = (uint16_t)(e[j] & 0xffffu);
      t[r][c + 2 * j + 1] = (uint16_t)(e[j] >> 16);
    }
  }
  __syncthreads();
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int nr = pass * 32 + (tid >> 3), kc = (tid & 7) * 8;  // output row n0 + nr, k0 + kc .. + 7
    if (n0 + nr >= N || k0 + kc >= K) continue;
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = (uint32_t)t[kc + 2 * j][nr] | ((uint32_t)t[kc + 2 * j + 1][nr] << 16);
    *reinterpret_cast<uint4*>(w + (n0 + nr) * K + k0 + kc) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

static inline unsigned nblocks(int64_t n, int t) { return (unsigned)((n + t - 1) / t); }

// Scoring head (src/server.py:37,57,129: mdl.head(hn[lastidx].float()).squeeze(-1), a Linear(H, 1) on fp32):
// scores[r] = sum_j float(hn[lastidx[r]][j]) * w[j] (+ bias). One wave per score: lane l takes the 8-column
// chunks l, l + 64, ... (16-byte coalesced loads), sums them in that order, then a fixed xor-butterfly across the
// wave; the result is the same on every run. An index outside [0, rows) gives NaN and reads nothing.
__global__ void __launch_bounds__(256) head_gemv_k(const uint16_t* __restrict__ hn, int64_t rows,
                                                   const int64_t* __restrict__ lastidx, int64_t R,
                                                   const float* __restrict__ w, const float* __restrict__ bias,
                                                   float* __restrict__ scores, int H) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;  // whole wave
  const int64_t row = lastidx[r];
  if (row < 0 || row >= rows) {
    if (lane == 0) scores[r] = __builtin_nanf("");
    return;
  }
  const uint16_t* src = hn + row * H;
  float acc = 0.f;
  for (int c = lane; c < H / 8; c += 64) {
    const uint4 v = *reinterpret_cast<const uint4*>(src + c * 8);
    const float4 w0 = *reinterpret_cast<const float4*>(w + c * 8);
    const float4 w1 = *reinterpret_cast<const float4*>(w + c * 8 + 4);
    acc = fmaf(bf2f(v.x & 0xffffu), w0.x, acc);
    acc = fmaf(bf2f(v.x >> 16), w0.y, acc);
    acc = fmaf(bf2f(v.y & 0xffffu), w0.z, acc);
    acc = fmaf(bf2f(v.y >> 16), w0.w, acc);
    acc = fmaf(bf2f(v.z & 0xffffu), w1.x, acc);
    acc = fmaf(bf2f(v.z >> 16), w1.y, acc);
    acc = fmaf(bf2f(v.w & 0xffffu), w1.z, acc);
    acc = fmaf(bf2f(v.w >> 16), w1.w, acc);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane == 0) scores[r] = acc + (bias != nullptr ? bias[0] : 0.f);
}

hipError_t launch_head_gemv(const uint16_t* hn, int64_t rows, const int64_t* lastidx, int64_t R, const float* w,
                            const float* bias, float* scores, int H, hipStream_t st) {
  hipLaunchKernelGGL(head_gemv_k, dim3(nblocks(R, 4)), dim3(256), 0, st, hn, rows, lastidx, R, w, bias, scores, H);
  return hipGetLastError();
}

hipError_t launch_reduce_bf16(const float* parts, int S, int64_t ps, uint16_t* y, int64_t ldy, int M, int N,
                              hipStream_t st) {
  const int64_t n = (int64_t)M * (N / 4);
  hipLaunchKernelGGL(reduce_bf16_k, dim3(nblocks(n, 256)), dim3(256), 0, st, parts, S, ps, y, ldy, M, N);
  return hipGetLastError();
}

hipError_t launch_reduce_silu(const float* parts, int S, int64_t ps, uint16_t* out, int64_t ldo, int M, int N,
                              hipStream_t st) {
  const int64_t n = (int64_t)M * (N / 8);
  hipLaunchKernelGGL(reduce_silu_k, dim3(nblocks(n, 256)), dim3(256), 0, st, parts, S, ps, out, ldo, M, N);
  return hipGetLastError();
}

hipError_t launch_add_rmsnorm(const uint16_t* x, const uint16_t* delta, const float* parts, int S, int64_t ps,
                              const float* w1, const int32_t* rowmask, float eps, uint16_t* h_out,
                              uint16_t* hn_out, int M, int H, hipStream_t st) {
  const int mode = parts != nullptr ? 2 : delta != nullptr ? 1 : 0;
  const bool hn = hn_out != nullptr;
#define OJX_RMS(MO, HV) \
  hipLaunchKernelGGL((add_rmsnorm_k<MO, HV>), dim3(M), dim3(H / 8), 0, st, x, delta, parts, S, ps, w1, rowmask, eps, \
                     h_out, hn_out, H)
  if (mode == 2) { if (hn) OJX_RMS(2, true); else OJX_RMS(2, false); }
  else if (mode == 1) { if (hn) OJX_RMS(1, true); else OJX_RMS(1, false); }
  else OJX_RMS(0, true);  // the host never asks for neither output
#undef OJX_RMS
  return hipGetLastError();
}

hipError_t launch_silu_mul(const uint16_t* gu, const uint16_t* tab, uint16_t* out, int M, int I, hipStream_t st) {
  const int64_t total8 = (int64_t)M * I / 8;
  hipLaunchKernelGGL(silu_mul_k, dim3(nblocks(total8, 256)), dim3(256), 0, st, gu, tab, out, I, total8);
  return hipGetLastError();
}

hipError_t launch_act_tables(uint16_t* silu_b, float* sig_f, hipStream_t st) {
  hipLaunchKernelGGL(act_tables_k, dim3(256), dim3(256), 0, st, silu_b, sig_f);
  return hipGetLastError();
}

hipError_t launch_pack_gate_up(const uint16_t* gate, const uint16_t* up, uint16_t* packed, int I, int K,
                               hipStream_t st) {
  const int64_t n = (int64_t)2 * I * (K / 8);
  hipLaunchKernelGGL(pack_gate_up_k, dim3(nblocks(n, 256)), dim3(256), 0, st, gate, up, packed, I, K);
  return hipGetLastError();
}

hipError_t launch_unsplit_weight(const uint16_t* wt, uint16_t* w, int64_t K, int64_t N, hipStream_t st) {
  hipLaunchKernelGGL(unsplit_weight_k, dim3((unsigned)((N + 63) / 64), (unsigned)((K + 63) / 64)), dim3(256), 0, st,
                     wt, w, K, N);
  return hipGetLastError();
}

hipError_t launch_pack_weight(const uint16_t* w, uint16_t* wp, int64_t N, int64_t K, hipStream_t st) {
  hipLaunchKernelGGL(pack_weight_k, dim3(nblocks(N * (K / 8), 256)), dim3(256), 0, st, w, wp, N, K);
  return hipGetLastError();
}

}  // namespace ojx
