// The two consumers of the in-projection output that forward_gtree calls by default: the full-attention prep and
// the linear-attention prep on the tree layout. Both are one workgroup per token row: the row is read once,
// finished in LDS, and written out with whole 8- or 16-byte vector stores.
#include "ojx_internal.h"

namespace ojx {

namespace {

// Sum over the 64 lanes of a wave (every lane gets the total).
__device__ __forceinline__ float wave_total(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ void unpack4(uint2 a, float (&v)[4]) {
  v[0] = bf2f(a.x & 0xffffu);
  v[1] = bf2f(a.x >> 16);
  v[2] = bf2f(a.y & 0xffffu);
  v[3] = bf2f(a.y >> 16);
}

}  // namespace

// ------------------------------------------------------------------------------------------------ full attention
// Reference behaviour: fullattn_prep2 (src/kernels.cu:302-355), called from forward_gtree as
// K.fullattn_prep2(proj, qw1, kw1, cos, sin, 1, N, HQ, HKV, D, eps) (src/fastmodel.py:462). proj [N, P] bf16 with
// P = HQ 2D + 2 HKV D; for token n:
//   q head h: x = proj[n][2hD .. 2hD+D), gate head h = proj[n][2hD+D .. 2hD+2D);
//   k head h: x = proj[n][2 HQ D + hD ..); v head h = proj[n][2 HQ D + HKV D + hD ..).
//   q and k: xn = bf16((x * rsqrt(sum x^2 / D + eps)) * w1[d]) with w1 = qw1 / kw1 [D] fp32, then on the first RD
//   dims the rotate-half RoPE: out = bf16(bf16(xn * cos[n][d]) + bf16(rh * sin[n][d])), rh = -xn[d + RD/2] for
//   d < RD/2 and xn[d - RD/2] for RD/2 <= d < RD; dims >= RD keep xn.
//   Outputs: qt [HQ, N, D], kt [HKV, N, D], vt [HKV, N, D] (head-major for attention) and gate [N, HQ D].
//
// Work layout: one wave per (token, head task), four tasks per workgroup. Task t of a token: t < HQ the q head t
// (the wave also copies gate head t), HQ <= t < HQ + HKV the k head t - HQ, then the v heads (copies). Lane l owns
// dims 4l .. 4l+3 (one 8-byte load, one 8-byte store: 512 contiguous bytes per wave). A q/k head's sum of squares
// is a 64-lane wave total; the normalised head goes to the wave's own 1 KB of LDS, from which each lane of the
// rotary part reads its four partner values xn[d -+ RD/2] (a wave-local exchange: no workgroup barrier).
__global__ void __launch_bounds__(256) fullattn_prep_k(const uint16_t* __restrict__ proj, int64_t N, int HQ, int HKV,
                                                       int RD, float eps, const float* __restrict__ qw1,
                                                       const float* __restrict__ kw1, const uint16_t* __restrict__ cosb,
                                                       const uint16_t* __restrict__ sinb, uint16_t* __restrict__ qt,
                                                       uint16_t* __restrict__ kt, uint16_t* __restrict__ vt,
                                                       uint16_t* __restrict__ gate) {
  constexpr int D = 256;
  __shared__ float4 xn_lds[4][D / 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int T = HQ + 2 * HKV, G = (T + 3) >> 2;  // tasks per token, workgroups per token
  const int64_t n = blockIdx.x / G;
  const int t = (int)(blockIdx.x - n * G) * 4 + wave;
  if (t >= T) return;  // whole wave; no workgroup barrier follows
  const int64_t P = (int64_t)(2 * HQ + 2 * HKV) * D;
  const uint16_t* row = proj + n * P;
  const int d0 = lane * 4;
  if (t >= HQ + HKV) {  // v head: a copy into [HKV, N, D]
    const int hv = t - HQ - HKV;
    *reinterpret_cast<uint2*>(vt + ((int64_t)hv * N + n) * D + d0) =
        *reinterpret_cast<const uint2*>(row + (int64_t)(2 * HQ + HKV) * D + hv * D + d0);
    return;
  }
  const bool isq = t < HQ;
  if (isq)  // gate head: a copy into [N, HQ D]
    *reinterpret_cast<uint2*>(gate + n * (int64_t)(HQ * D) + t * D + d0) =
        *reinterpret_cast<const uint2*>(row + (int64_t)t * 2 * D + D + d0);
  float x[4];
  unpack4(*reinterpret_cast<const uint2*>(row + (isq ? (int64_t)t * 2 * D : (int64_t)2 * HQ * D + (int64_t)(t - HQ) * D)
                                          + d0), x);
  float ss = x[0] * x[0];
  ss += x[1] * x[1];
  ss += x[2] * x[2];
  ss += x[3] * x[3];
  const float r = rsqrtf(wave_total(ss) / (float)D + eps);
  const float4 w = *reinterpret_cast<const float4*>((isq ? qw1 : kw1) + d0);
  float xn[4];
  xn[0] = rbf((x[0] * r) * w.x);
  xn[1] = rbf((x[1] * r) * w.y);
  xn[2] = rbf((x[2] * r) * w.z);
  xn[3] = rbf((x[3] * r) * w.w);
  float o[4] = {xn[0], xn[1], xn[2], xn[3]};
  if (RD > 0) {
    xn_lds[wave][lane] = make_float4(xn[0], xn[1], xn[2], xn[3]);
    // the wave's LDS writes are complete and visible to its own lanes before the partner reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (d0 < RD) {
      float cs[4], sn[4];
      unpack4(*reinterpret_cast<const uint2*>(cosb + n * RD + d0), cs);
      unpack4(*reinterpret_cast<const uint2*>(sinb + n * RD + d0), sn);
      const bool lo = d0 < RD / 2;
      const float4 pq = xn_lds[wave][(lo ? d0 + RD / 2 : d0 - RD / 2) >> 2];
      const float pv[4] = {pq.x, pq.y, pq.z, pq.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = rbf(rbf(xn[j] * cs[j]) + rbf((lo ? -pv[j] : pv[j]) * sn[j]));
    }
  }
  uint16_t* dst = isq ? qt + ((int64_t)t * N + n) * D : kt + ((int64_t)(t - HQ) * N + n) * D;
  *reinterpret_cast<uint2*>(dst + d0) = make_uint2(pack2(o[0], o[1]), pack2(o[2], o[3]));
}

hipError_t launch_fullattn_prep(const uint16_t* proj, int64_t N, int HQ, int HKV, int RD, float eps,
                                const float* qw1, const float* kw1, const uint16_t* cosb, const uint16_t* sinb,
                                uint16_t* qt, uint16_t* kt, uint16_t* vt, uint16_t* gate, hipStream_t st) {
  const int64_t G = (HQ + 2 * HKV + 3) / 4;
  hipLaunchKernelGGL(fullattn_prep_k, dim3((unsigned)(N * G)), dim3(256), 0, st, proj, N, HQ, HKV, RD, eps, qw1, kw1,
                     cosb, sinb, qt, kt, vt, gate);
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------ linear attention
// Reference behaviour: linattn_prep_dedup2 (src/kernels.cu:1176-1265), called from forward_gtree as
// K.linattn_prep_dedup2(proj, lay.hist, lay.rep_ptr, lay.rep_pos, lay.L2, convw, A_log, dt_bias, KD, VD, HV, HK, HD,
// rep_qk) (src/fastmodel.py:420,438). proj [N, P] bf16, P = C + VD + 2 HV with C = 2 KD + VD conv channels
// (q | k | v), then the z gate (VD, read later by the gated norm), then b [HV] and a [HV]. Each packed row n is
// computed once and written to every slot s = rep_pos[p], p in [rep_ptr[n], rep_ptr[n+1]) (the candidate paths that
// contain it); the slots of group N (rep_ptr[N] .. rep_ptr[N+1]) are the paths' end padding and receive zeros.
//   channel c: conv = sum_{i=0..3} convw[c][i] * proj[hist[n][i]][c], added in that order (hist[n] = the rows
//   t-3 .. t on the row's path, -1 = none); o = bf16(silu(conv)). q and k channels (c < 2 KD) are then
//   L2-normalised over their head of HD = 128 channels: bf16(o * (1 / sqrt(sum o^2 + 1e-6))).
//   head h < HV: beta = bf16(sigmoid(b_h)), g = -exp(A_log[h]) * softplus(a_h + dt_bias[h]) (fp32, softplus(x) = x
//   above 20), b and a read from row hist[n][3].
//   Outputs: q, k [R, HK RQ HD] (RQ = 1, or 3 = HV / HK copies of each head side by side), v [R, VD], g [R, HV] fp32,
//   beta [R, HV] bf16; R = rep_pos's length.
// Products of two bf16 values are exact in fp32, so the conv's sum order is the only one that fixes its bits; it is
// kept. The head sums of squares are added in another order than the reference's (one rounding step at most).
//
// Work layout: one workgroup of 8 waves (kLinThreads = 512 lanes) per packed row, grid = N rows + the padding
// groups.
//   1. conv + SiLU for all C channels (8 per lane per step, the four history rows and the 64 weight bytes as 16-byte
//      loads; 10240 channels take 2.5 steps), the bf16 results kept in an LDS copy of the row;
//   2. one q/k head per wave at a time, 2 channels per lane: wave-total sum of squares, scaled in place in LDS;
//      lanes below HV compute the gates into LDS meanwhile;
//   3. the finished row is written slot after slot: every 16-byte chunk of a slot's q | k | v row is one lane's
//      LDS read and global store, so each slot row goes out as one contiguous sweep; slot ids come in through
//      LDS, kLinThreads at a time (the first batch fetched before step 1).
// A padding group (the workgroups after the N row workgroups) writes zero rows to kPadSlots consecutive
// padding slots.
constexpr int kPadSlots = 8;

constexpr int kLinThreads = 512;

template <int RQ>
__global__ void __launch_bounds__(kLinThreads) linattn_prep_k(const uint16_t* __restrict__ proj, const int4* __restrict__ hist,
                                                     const int* __restrict__ rep_ptr, const int* __restrict__ rep_pos,
                                                     const uint16_t* __restrict__ convw,
                                                     const uint16_t* __restrict__ A_log,
                                                     const uint16_t* __restrict__ dt_bias, uint16_t* __restrict__ q,
                                                     uint16_t* __restrict__ k, uint16_t* __restrict__ v,
                                                     float* __restrict__ g, uint16_t* __restrict__ beta, int N, int KD,
                                                     int VD, int HV) {
  constexpr int HD = 128;
  extern __shared__ uint4 lds_raw[];
  const int C = 2 * KD + VD;
  const int64_t P = (int64_t)C + VD + 2 * HV;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = blockIdx.x;
  const bool pad = n >= N;
  const int4 hr = hist[min(n, N)];  // row N holds no history; issued beside the rep_ptr loads
  int p0, p1;
  if (!pad) {
    p0 = rep_ptr[n];
    p1 = rep_ptr[n + 1];
  } else {
    p0 = rep_ptr[N] + (n - N) * kPadSlots;
    p1 = min(rep_ptr[N + 1], p0 + kPadSlots);
  }
  if (p0 >= p1) return;  // uniform over the workgroup

  uint16_t* orow = reinterpret_cast<uint16_t*>(lds_raw);                 // [C] bf16 bits
  float* gl = reinterpret_cast<float*>(orow + C);                         // [HV] g
  uint16_t* bl = reinterpret_cast<uint16_t*>(gl + HV);                    // [HV] beta bits
  int* slot = reinterpret_cast<int*>(lds_raw) + (C * 2 + HV * 6 + 15) / 16 * 4;  // [kLinThreads] slot ids
  // the first batch of slot ids is fetched now, so that its latency overlaps the row's compute
  const int cnt0 = min(kLinThreads, p1 - p0);
  const int sid0 = tid < cnt0 ? rep_pos[p0 + tid] : 0;

  if (!pad) {
    const int rows[4] = {hr.x, hr.y, hr.z, hr.w};
    for (int c0 = tid * 8; c0 < C; c0 += kLinThreads * 8) {
      uint4 xr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xr[i] = rows[i] >= 0 ? *reinterpret_cast<const uint4*>(proj + (int64_t)rows[i] * P + c0)
                             : make_uint4(0u, 0u, 0u, 0u);
      const uint4* wp = reinterpret_cast<const uint4*>(convw + (int64_t)c0 * 4);  // [8 channels][4 taps]
      const uint4 wq[4] = {wp[0], wp[1], wp[2], wp[3]};
      const uint32_t* wv = &wq[0].x;
      uint32_t packed[4];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        float o2[2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int ch = j + jj;
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t* xw = &xr[i].x;
            const float xv = bf2f((xw[ch >> 1] >> ((ch & 1) * 16)) & 0xffffu);
            const int wi = ch * 4 + i;
            const float wf = bf2f((wv[wi >> 1] >> ((wi & 1) * 16)) & 0xffffu);
            acc += wf * xv;
          }
          o2[jj] = silu_f(acc);
        }
        packed[j >> 1] = pack2(o2[0], o2[1]);
      }
      *reinterpret_cast<uint4*>(orow + c0) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    }
    if (tid < HV) {
      const uint16_t* br = proj + (int64_t)hr.w * P + C + VD;
      bl[tid] = (uint16_t)f2bf(sigmoid_f(bf2f(br[tid])));
      const float xs = bf2f(br[HV + tid]) + bf2f(dt_bias[tid]);
      gl[tid] = -expf(bf2f(A_log[tid])) * (xs > 20.f ? xs : log1pf(expf(xs)));
    }
    __syncthreads();
    // q / k heads: one per wave at a time, channels 2 lane, 2 lane + 1
    for (int h = wave; h < 2 * KD / HD; h += kLinThreads / 64) {
      uint32_t* pr = reinterpret_cast<uint32_t*>(orow + h * HD) + lane;
      const uint32_t u = *pr;
      const float a = bf2f(u & 0xffffu), b = bf2f(u >> 16);
      float ss = a * a;
      ss += b * b;
      const float rs = 1.0f / sqrtf(wave_total(ss) + 1e-6f);
      *pr = pack2(a * rs, b * rs);
    }
  }
  __syncthreads();

  // scatter: chunk u of a slot row is q (u < QC), k (QC <= u < 2 QC) or v; q/k rows hold each head RQ times
  const int QC = RQ * KD / 8, VC = VD / 8, U = 2 * QC + VC;
  for (int base = p0; base < p1; base += kLinThreads) {
    const int cnt = min(kLinThreads, p1 - base);
    if (tid < cnt) slot[tid] = base == p0 ? sid0 : rep_pos[base + tid];
    __syncthreads();
    for (int j = 0; j < cnt; ++j) {
      const int64_t s = slot[j];
      for (int u = tid; u < U; u += kLinThreads) {
        uint4 val = make_uint4(0u, 0u, 0u, 0u);
        uint16_t* dst;
        int src;
        if (u < 2 * QC) {
          const bool isk = u >= QC;
          const int e = (u - (isk ? QC : 0)) * 8;  // element within the RQ KD row
          const int hk = e / (RQ * HD);
          src = (isk ? KD : 0) + hk * HD + (e - hk * RQ * HD) % HD;
          dst = (isk ? k : q) + s * (int64_t)(RQ * KD) + e;
        } else {
          const int e = (u - 2 * QC) * 8;
          src = 2 * KD + e;
          dst = v + s * (int64_t)VD + e;
        }
        if (!pad) val = *reinterpret_cast<const uint4*>(orow + src);
        *reinterpret_cast<uint4*>(dst) = val;
      }
      if (tid < HV) {
        g[s * HV + tid] = pad ? 0.f : gl[tid];
        beta[s * HV + tid] = pad ? (uint16_t)0 : bl[tid];
      }
    }
    __syncthreads();  // slot[] is refilled by the next batch
  }
}

hipError_t launch_linattn_prep(const uint16_t* proj, const int32_t* hist, const int32_t* rep_ptr,
                               const int32_t* rep_pos, int64_t N, int64_t R, const uint16_t* convw,
                               const uint16_t* A_log, const uint16_t* dt_bias, int KD, int VD, int HV, int RQ,
                               uint16_t* q, uint16_t* k, uint16_t* v, float* g, uint16_t* beta, hipStream_t st) {
  const int C = 2 * KD + VD;
  const size_t lds = (size_t)((C * 2 + HV * 6 + 15) / 16) * 16 + kLinThreads * sizeof(int);
  const dim3 grid((unsigned)(N + (R + kPadSlots - 1) / kPadSlots));
  if (RQ == 3)
    hipLaunchKernelGGL(linattn_prep_k<3>, grid, dim3(kLinThreads), lds, st, proj, reinterpret_cast<const int4*>(hist),
                       rep_ptr, rep_pos, convw, A_log, dt_bias, q, k, v, g, beta, (int)N, KD, VD, HV);
  else
    hipLaunchKernelGGL(linattn_prep_k<1>, grid, dim3(kLinThreads), lds, st, proj, reinterpret_cast<const int4*>(hist),
                       rep_ptr, rep_pos, convw, A_log, dt_bias, q, k, v, g, beta, (int)N, KD, VD, HV);
  return hipGetLastError();
}

}  // namespace ojx
