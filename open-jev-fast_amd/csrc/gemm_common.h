// Device helpers shared by the GEMM translation units: buffer-resource loads, LDS-only barrier and the fused
// fragment epilogue (bf16 store, fp32 partial, residual add, SiLU.mul of packed gate/up rows).
#pragma once
#include "ojx_internal.h"

namespace ojx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Buffer loads: the descriptor's byte range makes out-of-range lanes read zeros without a branch, so predicated
// tile loads stay in flight (a branch around each load would make the compiler drain the load queue at the join).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int32_t n = bytes > 0x7fffffffLL ? 0x7fffffff : (int32_t)(bytes < 0 ? 0 : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// Non-temporal load (cache-policy bit nt): for the weight stream, read once per call, so that it does not evict the
// activations every workgroup shares from L2. Measured on MI355X: a weight stream with the hint reaches 6.4 TB/s
// against 6.1 without, and streams that mix weights and L2-resident activations run about 9% faster.
__device__ __forceinline__ uint4 bload_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}
constexpr uint32_t kOOB = 0x80000000u;  // an offset past every descriptor's range: the load returns zeros

// Wait until at most N of this wave's vector-memory operations are outstanding (LDS-DMA loads, coherent stores).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Cache policy of device-coherent accesses (sc0 sc1): stores written through to the level every XCD reads, loads
// served from there. For data exchanged between workgroups of one launch, which may run on different XCDs whose L2s
// are not coherent with each other.
constexpr int kCoh = 1 | 16;

// Sum over the S fp32 planes (plane stride ps elements) of the float4 at byte offset off, in ascending plane order,
// with device-coherent loads; the loads go out eight planes at a time (indices clamped, extras not added).
__device__ __forceinline__ f32x4 sum_planes_coh(__amdgpu_buffer_rsrc_t r, uint32_t off, int S, int64_t ps) {
  f32x4 a = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCoh));
  for (int s0 = 1; s0 < S; s0 += 8) {
    f32x4 c[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t s = s0 + u < S ? s0 + u : S - 1;
      c[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(off + s * ps * 4), 0, kCoh));
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s0 + u < S) a += c[u];
  }
  return a;
}

// 16-byte global -> LDS DMA: lane i of the wave writes lds + 16 i. (Kept out of the kernel templates: written
// inline there, the address-space cast stops the host pass from emitting the kernels' launch stubs.)
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// The same DMA with the non-temporal hint: the lines are not kept in L2 for reuse. For operands that are read once
// per call (the weight stream), so that they do not evict operands that other workgroups are about to read.
__device__ __forceinline__ void dma16_nt(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 2);
}

// The LDS DMA with a wave-uniform byte offset (soffset) added to the lane's offset: loop-invariant lane offsets in
// VGPRs, the per-stage part in an SGPR, so that issuing a DMA costs no vector instruction.
__device__ __forceinline__ void dma16s(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma16s_nt(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 2);
}

// Workgroup barrier that orders LDS only. __syncthreads() is a full workgroup fence, which on gfx9 waits for every
// outstanding global load (vmcnt(0)) and would drain the weight prefetch queue at each x-tile handoff.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}


// Counts the calling workgroup in *ctr (agent scope) after all its threads' device-coherent stores have completed,
// and returns on every thread whether it was the last of `expect` arrivals; the last re-arms the counter. No
// workgroup waits for another: the last one does the follow-up work, so the launch cannot deadlock whatever order
// or residency its workgroups get.
__device__ __forceinline__ bool ol_arrive(uint32_t* ctr, uint32_t expect) {
  __shared__ uint32_t last;
  wait_vmcnt<0>();  // this thread's stores are at the coherent level
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old + 1 == expect ? 1u : 0u;
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return last != 0u;
}

// After each split of tile (tn, tm) has stored its fp32 plane (device-coherent stores): the last split to arrive
// sums the tile's S planes in split order, the arithmetic and order of reduce_bf16_k / reduce_silu_k /
// add_rmsnorm_k (epilogue.hip), and stores the epilogue's result. With the residual epilogue and hn it also stores
// the tile's per-row sums of h^2 (over its BN columns, in column order), and the last tile of the M block to
// arrive normalises the block's rows: r = rsqrt(sum over the N tiles, in tile order, / N + eps), hn = bf16((h r) w1),
// zero on masked rows. The bits of y, out and h equal the two-launch path's; hn's sum of squares is added in
// another order than add_rmsnorm_k's (a rounding step at most). `lds` is the kernel's operand LDS, free by now.
template <int BN, int BM, int NT, int URMAX = 1>
__device__ __forceinline__ void ol_epilogue(const GemmParams& p, const int epi, const int tn, const int tm, float* lds) {
  const int M = p.M, N = p.N, S = p.splits;
  if (!ol_arrive(p.ol_tiles + tn * p.tiles_m + tm, (uint32_t)S)) return;
  const int n0 = tn * BN, m0 = tm * BM, tid = threadIdx.x;
  const int64_t ps = (int64_t)M * N;
  const __amdgpu_buffer_rsrc_t rsP = make_rsrc(p.ol_parts, S * ps * 4);
  const bool norm = epi == EPI_RESID && p.hn != nullptr;  // the RMSNorm fold (one_launch = 2)
  // h of the residual epilogue, read back by the row pass (possibly on another XCD): one descriptor over [M, ldo]
  const __amdgpu_buffer_rsrc_t rsH = make_rsrc(p.out, (int64_t)M * p.ldo * 2);
  // groups of 4 columns (8 for the SiLU.mul pairs: 4 gate then 4 up columns give 4 outputs)
  const int gw = epi == EPI_SILU ? 8 : 4, gpr = BN / gw, nitem = BM * gpr;
  // the epilogue of one item from its plane sums (a; u: the up columns of a SiLU.mul pair); returns its sum of h^2
  auto finish = [&](const int m, const int n, const f32x4 a, const f32x4 u) -> float {
    float hsq = 0.f;
    if (epi == EPI_SILU) {
      uint16_t* dst = reinterpret_cast<uint16_t*>(p.out) + (int64_t)m * p.ldo + (n >> 1);
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = f2bf(rbf(silu_f(rbf(a[e]))) * rbf(u[e]));
      *reinterpret_cast<uint2*>(dst) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
    } else {
      uint16_t* dst = reinterpret_cast<uint16_t*>(p.out) + (int64_t)m * p.ldo + n;
      if (epi == EPI_RESID) {
        const uint2 rr = *reinterpret_cast<const uint2*>(p.res + (int64_t)m * p.ldr + n);
        const float rv[4] = {bf2f(rr.x & 0xffffu), bf2f(rr.x >> 16), bf2f(rr.y & 0xffffu), bf2f(rr.y >> 16)};
        float h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = rbf(rv[e] + rbf(a[e]));
        hsq = h[0] * h[0];
        hsq += h[1] * h[1];
        hsq += h[2] * h[2];
        hsq += h[3] * h[3];
        const uint2 hv = make_uint2(pack2(h[0], h[1]), pack2(h[2], h[3]));
        if (norm)
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, hv), rsH,
                                                (uint32_t)(((int64_t)m * p.ldo + n) * 2), 0, kCoh);
        else
          *reinterpret_cast<uint2*>(dst) = hv;
      } else {
        *reinterpret_cast<uint2*>(dst) = make_uint2(pack2(a[0], a[1]), pack2(a[2], a[3]));
      }
    }
    return hsq;
  };
  constexpr int UR0 = (BM * BN / 4 + NT - 1) / NT;
  constexpr int UR = UR0 < URMAX ? UR0 : URMAX;
  if constexpr (UR == 1) {
    // one item at a time, its planes loaded 8 at a time
    for (int it = tid; it < nitem; it += NT) {
      const int mi = it / gpr, n = n0 + (it - mi * gpr) * gw, m = m0 + mi;
      float hsq = 0.f;
      if (m < M && n < N) {
        const uint32_t off = (uint32_t)(((int64_t)m * N + n) * 4);
        const f32x4 a = sum_planes_coh(rsP, off, S, ps);
        const f32x4 u = epi == EPI_SILU ? sum_planes_coh(rsP, off + 16, S, ps) : a;
        hsq = finish(m, n, a, u);
      }
      if (norm) lds[it] = hsq;
    }
  } else {
    // UR items per thread and pass, the plane loads of all of them issued before adding (PB planes at a time, at
    // most 16 loads in flight): a round trip per PB planes rather than one per item; planes still summed in order
    constexpr int PB = 16 / (2 * UR) > 0 ? 16 / (2 * UR) : 1;
    for (int it0 = 0; it0 < nitem; it0 += UR * NT) {
      f32x4 ag[UR], au[UR];
      uint32_t off[UR];
      bool live[UR];
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        const int it = it0 + u * NT + tid, mi = it / gpr, n = n0 + (it - mi * gpr) * gw, m = m0 + mi;
        live[u] = it < nitem && m < M && n < N;
        off[u] = live[u] ? (uint32_t)(((int64_t)m * N + n) * 4) : 0u;
      }
      for (int s0 = 0; s0 < S; s0 += PB) {
        f32x4 cg[PB][UR], cu[PB][UR];
#pragma unroll
        for (int j = 0; j < PB; ++j)
#pragma unroll
          for (int u = 0; u < UR; ++u) {
            const uint32_t o = (uint32_t)(off[u] + (int64_t)min(s0 + j, S - 1) * ps * 4);
            cg[j][u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsP, o, 0, kCoh));
            if (epi == EPI_SILU)
              cu[j][u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsP, o + 16, 0, kCoh));
          }
#pragma unroll
        for (int j = 0; j < PB; ++j)
#pragma unroll
          for (int u = 0; u < UR; ++u) {
            if (s0 + j >= S) continue;
            ag[u] = s0 + j == 0 ? cg[j][u] : ag[u] + cg[j][u];
            if (epi == EPI_SILU) au[u] = s0 + j == 0 ? cu[j][u] : au[u] + cu[j][u];
          }
      }
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        const int it = it0 + u * NT + tid, mi = it / gpr, n = n0 + (it - mi * gpr) * gw, m = m0 + mi;
        const float hsq = live[u] ? finish(m, n, ag[u], epi == EPI_SILU ? au[u] : ag[u]) : 0.f;
        if (norm && it < nitem) lds[it] = hsq;
      }
    }
  }
  if (!norm) return;
  // the tile's row sums of h^2, in column order
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rsS = make_rsrc(p.ol_ss, (int64_t)p.tiles_n * M * 4);
  for (int r = tid; r < BM && m0 + r < M; r += NT) {  // a tile may have more rows than threads (BM > NT)
    float s = 0.f;
    for (int c = 0; c < gpr; ++c) s += lds[r * gpr + c];
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, s), rsS, (uint32_t)(((int64_t)tn * M + m0 + r) * 4), 0, kCoh);
  }
  if (!ol_arrive(p.ol_blocks + tm, (uint32_t)p.tiles_n)) return;
  // the block's row pass over all N columns
  float* rr = lds;  // [BM] 1 / rms
  for (int r = tid; r < BM && m0 + r < M; r += NT) {
    float s = 0.f;
    for (int t0 = 0; t0 < p.tiles_n; t0 += 16) {  // 16 loads in flight, added in tile order
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u)
        v[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             rsS, (uint32_t)(((int64_t)min(t0 + u, p.tiles_n - 1) * M + m0 + r) * 4),
                                             0, kCoh));
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (t0 + u < p.tiles_n) s += v[u];
    }
    rr[r] = rsqrtf(s / (float)N + p.eps);
  }
  __syncthreads();
  // 8 items (8 columns each) per thread per batch: the h loads of a batch go out together
  const int cpr = N >> 3, items = (min(M, m0 + BM) - m0) * cpr;
  constexpr int U = 8;
  for (int i0 = 0; i0 < items; i0 += NT * U) {
    uint4 hv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int it = i0 + u * NT + tid, mi = it / cpr, n = (it - mi * cpr) * 8;
      hv[u] = it < items ? __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                               rsH, (uint32_t)(((int64_t)(m0 + mi) * p.ldo + n) * 2), 0, kCoh))
                         : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int it = i0 + u * NT + tid;
      if (it >= items) continue;
      const int mi = it / cpr, n = (it - mi * cpr) * 8, m = m0 + mi;
      const float4 wa = *reinterpret_cast<const float4*>(p.w1 + n), wb = *reinterpret_cast<const float4*>(p.w1 + n + 4);
      const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
      const uint32_t hw[4] = {hv[u].x, hv[u].y, hv[u].z, hv[u].w};
      const bool keep = p.rowmask == nullptr || p.rowmask[m] != 0;
      const float r = rr[mi];
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = keep ? (bf2f((hw[j >> 1] >> ((j & 1) * 16)) & 0xffffu) * r) * wv[j] : 0.f;
      *reinterpret_cast<uint4*>(p.hn + (int64_t)m * N + n) =
          make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
    }
  }
}

// Epilogue of 4 consecutive outputs y[m][n .. n+3] (n a multiple of 4) held by one lane. For the fused SiLU.mul,
// `u` is the partner lane's values: packed W_gu rows come in blocks of 8 (4 gate rows, then the 4 up rows of the
// same columns), so a lane holding gate columns (`gate` true) finds its up columns in the partner lane.
__device__ __forceinline__ void store4(const GemmParams& p, const int epi, const int z, const int m, const int n,
                                       const bool gate, const f32x4 v, const f32x4 u) {
  if (m >= p.M || n >= p.N) return;
  if (epi == EPI_SILU) {
    if (!gate) return;
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = f2bf(rbf(silu_f(rbf(v[e]))) * rbf(u[e]));
    uint16_t* dst = reinterpret_cast<uint16_t*>(p.out) + (int64_t)m * p.ldo + (n >> 1);
    *reinterpret_cast<uint2*>(dst) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
  } else if (epi == EPI_F32) {
    float* dst = reinterpret_cast<float*>(p.out) + z * p.part_stride + (int64_t)m * p.ldo + n;
    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint32_t o[4];
    if (epi == EPI_RESID) {
      const uint2 rr = *reinterpret_cast<const uint2*>(p.res + (int64_t)m * p.ldr + n);
      const float rv[4] = {bf2f(rr.x & 0xffffu), bf2f(rr.x >> 16), bf2f(rr.y & 0xffffu), bf2f(rr.y >> 16)};
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = f2bf(rv[e] + rbf(v[e]));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = f2bf(v[e]);
    }
    uint16_t* dst = reinterpret_cast<uint16_t*>(p.out) + (int64_t)m * p.ldo + n;
    *reinterpret_cast<uint2*>(dst) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
  }
}

__device__ __forceinline__ f32x4 shfl4(const f32x4 v, int mask) {
  return f32x4{__shfl_xor(v[0], mask), __shfl_xor(v[1], mask), __shfl_xor(v[2], mask), __shfl_xor(v[3], mask)};
}

// Fused SiLU.mul of one fragment with the work split over both lanes of each gate/up pair: after the exchange the
// gate lane (even lane group, gate columns n .. n+3) and its partner (up columns of the same outputs) each hold all
// eight values, and each computes two of the four outputs, so no lane idles through the exp and the division.
// Output column of lane: (gate column) / 2, + 2 for the partner.
__device__ __forceinline__ void store_silu_pair(const GemmParams& p, const int m, const int n, const bool gate,
                                                const f32x4 v, const f32x4 u) {
  const int ng = gate ? n : n - 4;  // the pair's gate column
  if (m >= p.M || ng >= p.N) return;
  const float g0 = gate ? v[0] : u[2], g1 = gate ? v[1] : u[3];
  const float u0 = gate ? u[0] : v[2], u1 = gate ? u[1] : v[3];
  const uint32_t o0 = f2bf(rbf(silu_f(rbf(g0))) * rbf(u0));
  const uint32_t o1 = f2bf(rbf(silu_f(rbf(g1))) * rbf(u1));
  uint16_t* dst = reinterpret_cast<uint16_t*>(p.out) + (int64_t)m * p.ldo + (ng >> 1) + (gate ? 0 : 2);
  *reinterpret_cast<uint32_t*>(dst) = o0 | (o1 << 16);
}

// Epilogue of one 16x16 accumulator fragment: lane holds v[e] = y[m][n + e]; lane group lg = lane / 16.
__device__ __forceinline__ void store_tile(const GemmParams& p, const int epi, const int z, const int m, const int n,
                                           const int lg, const f32x4 v) {
  if (epi == EPI_SILU) {
    const f32x4 u = shfl4(v, 16);  // all lanes take part in the exchange
    store_silu_pair(p, m, n, (lg & 1) == 0, v, u);
    return;
  }
  store4(p, epi, z, m, n, true, v, v);
}


}  // namespace ojx

namespace ojx {
// Persistent stream-K family (gemm_sk.hip; instantiated there for the shapes of the tile table).
template <int FN, int FM, int WN, int WM>
__global__ void gemm_sk_kernel(const GemmParams p, const int epi);
template <int FN, int FM, int WN, int WM>
__global__ void gemm_sk_fixup_kernel(const GemmParams p, const int epi);
template <int FN, int FM, int WN, int WM>
__global__ void gemm_sk_fixup_rmsnorm_kernel(const GemmParams p, const float* w1, const int32_t* rowmask, float eps,
                                             uint16_t* hn_out);
// Its dynamic LDS: 3 stage buffers of (BN + BM) rows x 128 B where they fit in 160 KiB, else 2 (or 3 W + 2 x).
constexpr int sk_nbuf(int BN, int BM) { return 3 * (BN + BM) * 128 <= 160 * 1024 ? 3 : 2; }
// with 2 stage buffers: a ring of 3 W stages beside 2 x stages (W DMAs a stage further ahead) where that fits
// and W is the larger part of a stage (measured 3-6% faster on 256 x 192; 2-6% slower on 256 x 256 and 192 x 288)
constexpr bool sk_asym(int BN, int BM) {
  return sk_nbuf(BN, BM) == 2 && BM < BN && (3 * BN + 2 * BM) * 128 <= 160 * 1024;
}
constexpr int sk_lds(int BN, int BM) {
  return sk_asym(BN, BM) ? (3 * BN + 2 * BM) * 128 : sk_nbuf(BN, BM) * (BN + BM) * 128;
}
// K-interleaved wave pairs (gemm_kx.hip): BN x BM = 16 FW x 16 (4 FX + XE), 8 waves, x ring of XD stages.
template <int FW, int FX, int XE, int XD>
__global__ void gemm_kx_kernel(const GemmParams p, const int epi);
}  // namespace ojx
