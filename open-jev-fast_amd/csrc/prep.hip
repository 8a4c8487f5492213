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
// Two (token, head task) pairs per wave64, 32 lanes each with 8 consecutive dims (one 16-byte load and store per
// lane, D = 256): the row's sum of squares is a butterfly over the 32 lanes, and the RoPE partner of lane l is lane
// l ^ (RD / 16), because dims d and d +- RD/2 sit RD/16 lanes apart and RD/16 is a power of two below 32
// (RD = 16 .. 256).
#include "ojx_internal.h"

namespace ojx {

namespace {

__device__ __forceinline__ void unpack8(uint4 a, float (&v)[8]) {
  const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf2f(w[i] & 0xffffu);
    v[2 * i + 1] = bf2f(w[i] >> 16);
  }
}

}  // namespace

__global__ void __launch_bounds__(256) fullattn_prep_k(const uint16_t* __restrict__ proj, int64_t N, int HQ, int HKV,
                                                       int RD, float eps, const float* __restrict__ qw1,
                                                       const float* __restrict__ kw1, const uint16_t* __restrict__ cosb,
                                                       const uint16_t* __restrict__ sinb, uint16_t* __restrict__ qt,
                                                       uint16_t* __restrict__ kt, uint16_t* __restrict__ vt,
                                                       uint16_t* __restrict__ gate) {
  constexpr int D = 256;
  const int lane = threadIdx.x & 31;
  const int ntask = HQ + 2 * HKV;
  const int64_t wid = (int64_t)blockIdx.x * (blockDim.x >> 5) + (threadIdx.x >> 5);
  if (wid >= N * ntask) return;  // whole 32-lane halves leave together
  const int64_t n = wid / ntask;
  const int task = (int)(wid - n * ntask);
  const int64_t P = (int64_t)(2 * HQ + 2 * HKV) * D;
  const uint16_t* row = proj + n * P;
  const int d0 = lane * 8;
  if (task >= HQ + HKV) {  // v head: a copy into [HKV, N, D]
    const int h = task - HQ - HKV;
    *reinterpret_cast<uint4*>(vt + ((int64_t)h * N + n) * D + d0) =
        *reinterpret_cast<const uint4*>(row + 2 * HQ * D + HKV * D + h * D + d0);
    return;
  }
  const bool isq = task < HQ;
  const int h = isq ? task : task - HQ;
  if (isq)  // gate head: a copy into [N, HQ D]
    *reinterpret_cast<uint4*>(gate + n * (int64_t)(HQ * D) + h * D + d0) =
        *reinterpret_cast<const uint4*>(row + (int64_t)h * 2 * D + D + d0);
  float x[8];
  unpack8(*reinterpret_cast<const uint4*>(row + (isq ? (int64_t)h * 2 * D : 2 * HQ * D + (int64_t)h * D) + d0), x);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float r = rsqrtf(ss / (float)D + eps);
  const float* w1 = (isq ? qw1 : kw1) + d0;
  const float4 wa = *reinterpret_cast<const float4*>(w1), wb = *reinterpret_cast<const float4*>(w1 + 4);
  const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
  float nv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) nv[j] = rbf((x[j] * r) * wv[j]);
  const int hl = RD >> 4;  // partner lane distance
  float pv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) pv[j] = __shfl_xor(nv[j], hl);
  float out[8];
  if (d0 < RD) {
    float c[8], sn[8];
    unpack8(*reinterpret_cast<const uint4*>(cosb + n * RD + d0), c);
    unpack8(*reinterpret_cast<const uint4*>(sinb + n * RD + d0), sn);
    const bool lo = d0 < RD / 2;
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = rbf(rbf(nv[j] * c[j]) + rbf((lo ? -pv[j] : pv[j]) * sn[j]));
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = nv[j];
  }
  uint16_t* dst = isq ? qt : kt;
  *reinterpret_cast<uint4*>(dst + ((int64_t)h * N + n) * D + d0) =
      make_uint4(pack2(out[0], out[1]), pack2(out[2], out[3]), pack2(out[4], out[5]), pack2(out[6], out[7]));
}

hipError_t launch_fullattn_prep(const uint16_t* proj, int64_t N, int HQ, int HKV, int RD, float eps,
                                const float* qw1, const float* kw1, const uint16_t* cosb, const uint16_t* sinb,
                                uint16_t* qt, uint16_t* kt, uint16_t* vt, uint16_t* gate, hipStream_t st) {
  const int64_t halves = N * (HQ + 2 * HKV);
  hipLaunchKernelGGL(fullattn_prep_k, dim3((unsigned)((halves + 7) / 8)), dim3(256), 0, st, proj, N, HQ, HKV, RD, eps,
                     qw1, kw1, cosb, sinb, qt, kt, vt, gate);
  return hipGetLastError();
}

// Linear-attention prep on the tree layout: the consumer of the linear-attention layers' in-projection.
//
// Reference: linattn_prep_dedup2_k (src/kernels.cu:1176-1265), called from forward_gtree as
// K.linattn_prep_dedup2(proj, lay.hist, lay.rep_ptr, lay.rep_pos, lay.L2, convw, A_log, dt_bias, KD, VD, HV, HK, HD,
// rep_qk) (src/fastmodel.py:420,438). proj [N, P] bf16, P = C + VD + 2 HV with C = 2 KD + VD conv channels
// (q | k | v), then the z gate (VD, read later by the gated norm), then b [HV] and a [HV]. Each packed row n is
// computed once and written to every slot s = rep_pos[p], p in [rep_ptr[n], rep_ptr[n+1]) (the candidate paths that
// contain it); the slots of group N (rep_ptr[N] .. rep_ptr[N+1]) are the paths' end padding and receive zeros.
//   channel c: conv = sum_{i=0..3} convw[c][i] * proj[hist[n][i]][c] in that order (hist[n] = the rows t-3 .. t on
//   the row's path, -1 = none), o = bf16(silu(conv)); q and k channels (c < 2 KD) are then L2-normalised over their
//   head of HD = 128 channels: o * (1 / sqrt(sum o^2 + 1e-6)), the sum added by a butterfly over 16 lanes of 8
//   channels each (xor 8, 4, 2, 1, each lane's 8 squares added in order first), and rounded to bf16.
//   head h < HV: beta = bf16(sigmoid(b_h)), g = -exp(A_log[h]) * softplus(a_h + dt_bias[h]) (fp32, softplus(x) = x
//   above 20).
//   Outputs: q, k [R, RQ HK HD] (RQ = 1, or 3 = HV / HK copies of each head side by side), v [R, VD], g [R, HV] fp32,
//   beta [R, HV] bf16; R = rep_pos's length.
//
// Layout of the work: a workgroup of 256 lanes takes 2048 channels of one packed row (each lane 8 consecutive
// channels, one 16-byte load per history row, 16 lanes = one q/k head), computes them once and stores them to each of
// the row's slots (a wave writes 1 KB contiguous per slot). Workgroups past the N packed rows write the
// end-padding slots, 16 slots each. Products of two bf16 values are exact in fp32, so the conv's sum is the only rounding order that
// matters, and it is kept.
template <int RQ>
__global__ void __launch_bounds__(256) linattn_prep_k(const uint16_t* __restrict__ proj, const int4* __restrict__ hist,
                                                     const int* __restrict__ rep_ptr, const int* __restrict__ rep_pos,
                                                     const uint16_t* __restrict__ convw,
                                                     const uint16_t* __restrict__ A_log,
                                                     const uint16_t* __restrict__ dt_bias, uint16_t* __restrict__ q,
                                                     uint16_t* __restrict__ k, uint16_t* __restrict__ v,
                                                     float* __restrict__ g, uint16_t* __restrict__ beta, int N, int KD,
                                                     int VD, int HV) {
  constexpr int HD = 128;
  const int C = 2 * KD + VD;
  const int64_t P = (int64_t)C + VD + 2 * HV;
  // plain row-major numbering: an XCD-contiguous run of rows was measured slower (the prompt rows, written to
  // every path, then pile onto one XCD)
  const int n = blockIdx.y, bx = blockIdx.x;
  const bool pad = n >= N;
  int p0, p1;
  if (!pad) {
    p0 = rep_ptr[n];
    p1 = rep_ptr[n + 1];
  } else {
    p0 = rep_ptr[N] + (n - N) * 16;
    p1 = min(rep_ptr[N + 1], p0 + 16);
  }
  if (p0 >= p1) return;
  const int4 hr = pad ? make_int4(-1, -1, -1, -1) : hist[n];
  const int tid = threadIdx.x;
  const bool gate_lane = bx == 0 && tid < HV;  // per-head gates
  float bv = 0.f, gv = 0.f;
  if (gate_lane && !pad) {
    const uint16_t* row = proj + (int64_t)hr.w * P + C + VD;
    bv = sigmoid_f(bf2f(row[tid]));
    const float xs = bf2f(row[HV + tid]) + bf2f(dt_bias[tid]);
    gv = -expf(bf2f(A_log[tid])) * (xs > 20.f ? xs : log1pf(expf(xs)));
  }
  const uint16_t bb = (uint16_t)f2bf(bv);
  const int c0 = (bx * 256 + tid) * 8;
  const bool live = c0 < C;  // C is a multiple of 128: a 16-lane head group is either all in or all out
  const bool isqk = c0 < 2 * KD;
  uint4 ov = make_uint4(0u, 0u, 0u, 0u);
  if (live && !pad) {
    const int rows[4] = {hr.x, hr.y, hr.z, hr.w};
    uint4 xr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      xr[i] = rows[i] >= 0 ? *reinterpret_cast<const uint4*>(proj + (int64_t)rows[i] * P + c0) : make_uint4(0, 0, 0, 0);
    uint4 wr[4];  // convw[c0 .. c0+8)[0..4): 64 contiguous bytes
#pragma unroll
    for (int u = 0; u < 4; ++u) wr[u] = *reinterpret_cast<const uint4*>(convw + (int64_t)c0 * 4 + u * 8);
    const uint32_t* xw[4] = {&xr[0].x, &xr[1].x, &xr[2].x, &xr[3].x};
    const uint32_t* ww = &wr[0].x;
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t xb = (xw[i][j >> 1] >> ((j & 1) * 16)) & 0xffffu;
        const uint32_t wb = (ww[(j * 4 + i) >> 1] >> (((j * 4 + i) & 1) * 16)) & 0xffffu;
        acc += bf2f(wb) * bf2f(xb);
      }
      o[j] = rbf(silu_f(acc));
    }
    if (isqk) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += o[j] * o[j];
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
      const float rs = 1.0f / sqrtf(ss + 1e-6f);
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = o[j] * rs;
    }
    ov = make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
  }
  // destination of this lane's 8 channels within a slot's row
  uint16_t* dst;
  int64_t rowlen;
  if (isqk) {
    const int cc = c0 < KD ? c0 : c0 - KD;
    const int hk = cc / HD;
    dst = (c0 < KD ? q : k) + (int64_t)hk * RQ * HD + (cc - hk * HD);
    rowlen = (int64_t)RQ * KD;
  } else {
    dst = v + (c0 - 2 * KD);
    rowlen = VD;
  }
  // The row's slots, staged through LDS 256 at a time: one coalesced load, then every lane reads the slot ids as
  // LDS broadcasts (independent reads the compiler can issue ahead, instead of a chain of dependent scalar loads).
  __shared__ int slot[256];
  for (int base = p0; base < p1; base += 256) {
    const int cnt = min(256, p1 - base);
    if (tid < cnt) slot[tid] = rep_pos[base + tid];
    __syncthreads();
    if (gate_lane)
      for (int j = 0; j < cnt; ++j) {
        const int64_t sp = slot[j];
        beta[sp * HV + tid] = bb;
        g[sp * HV + tid] = gv;
      }
    if (live)
      for (int j = 0; j < cnt; ++j) {
        uint16_t* o = dst + (int64_t)slot[j] * rowlen;
#pragma unroll
        for (int r = 0; r < (isqk ? RQ : 1); ++r) *reinterpret_cast<uint4*>(o + r * HD) = ov;
      }
    __syncthreads();
  }
}

hipError_t launch_linattn_prep(const uint16_t* proj, const int32_t* hist, const int32_t* rep_ptr,
                               const int32_t* rep_pos, int64_t N, int64_t R, const uint16_t* convw,
                               const uint16_t* A_log, const uint16_t* dt_bias, int KD, int VD, int HV, int RQ,
                               uint16_t* q, uint16_t* k, uint16_t* v, float* g, uint16_t* beta, hipStream_t st) {
  const int C = 2 * KD + VD;
  const dim3 grid((unsigned)((C / 8 + 255) / 256), (unsigned)(N + (R + 15) / 16));
  if (RQ == 3)
    hipLaunchKernelGGL(linattn_prep_k<3>, grid, dim3(256), 0, st, proj, reinterpret_cast<const int4*>(hist), rep_ptr,
                       rep_pos, convw, A_log, dt_bias, q, k, v, g, beta, (int)N, KD, VD, HV);
  else
    hipLaunchKernelGGL(linattn_prep_k<1>, grid, dim3(256), 0, st, proj, reinterpret_cast<const int4*>(hist), rep_ptr,
                       rep_pos, convw, A_log, dt_bias, q, k, v, g, beta, (int)N, KD, VD, HV);
  return hipGetLastError();
}

}  // namespace ojx
