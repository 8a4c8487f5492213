// Skinny-M weight-streaming GEMM with the K split over the waves of one workgroup (family 7).
//
// At M <= 32 a projection is a weight stream: every W byte is used by at most 32 x rows, so the call is bound by
// HBM (N K 2 bytes) and the only question is how to keep enough weight loads in flight. The split-K plans of the
// other families get their parallelism from the grid (one workgroup per (W tile, K split)), which costs a second
// launch that sums fp32 planes through memory (about 4.6 us per call on MI355X, of a 12-28 us call). Here the K
// split stays inside the workgroup instead:
//
//   * Workgroup = NW waves over one tile of 16 FW W rows x 16 FM x rows; wave w takes a contiguous run of the
//     tile's 64-k stages (the runs differ by at most one stage) and multiplies all FW x FM fragments over it.
//   * Loads cover whole 128-byte lines (lane l: row l / 8 of an 8-row group, 16-byte chunk l % 8); each wave
//     passes its stage through its own LDS region to get the MFMA operand layout, without a workgroup barrier.
//     In the packed weight layout ([K/64][N/16][16][64], ojx_pack_weight) a tile's stage is one contiguous run.
//   * A ring of D stages of loads in flight per wave (the slot index is a compile-time constant: the stage loop
//     is unrolled by D). Stages past the wave's run re-read a stage of the run and skip their MFMAs (a
//     wave-uniform branch), so no load sits behind a branch. A split must be whole 64-k stages.
//   * At the end the NW partial tiles meet in LDS and are summed in wave order (deterministic), then the fused
//     epilogue of the other families stores them (bf16, fp32 split plane, residual, SiLU.mul pair).
//
// One launch per call and no workspace for every epilogue; the residual projection's RMSNorm still needs whole
// rows (all N tiles) and runs as the row kernel that re-reads h, as for the other whole-tile plans.
// Measured on the projection shapes at M = 1-32: 5-12% slower than the split-K plans (N / 16 fragments do not
// divide evenly over 256 CUs, where a grid split divides them finer), so the offline tuner picks none of these
// tiles; they stay candidates for other shapes.
#include "gemm_common.h"

namespace ojx {

template <int FW, int FM, int NW, int D>
__global__ void __launch_bounds__(64 * NW) gemm_sw_kernel(const GemmParams p, const int epi) {
  constexpr int BN = 16 * FW, BM = 16 * FM;
  constexpr int NF = FW * FM;
  constexpr int RW = BN / 8, RX = BM / 8;  // full-line loads per stage: 8 rows x 128 B each
  constexpr int SLOT = (BN + BM) * 128;    // bytes of one stage in a wave's LDS region
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // [NW][SLOT]; the reduction reuses it

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15, lg = lane >> 4;

  const int b = blockIdx.x;
  const int tm = b % p.tiles_m;
  const int t2 = b / p.tiles_m;
  const int z = t2 % p.splits;
  const int tn = t2 / p.splits;
  const int n0 = tn * BN, m0 = tm * BM;
  const int kb = z * p.kchunk;
  const int ke = min(p.K, kb + p.kchunk);
  const int nst = ke > kb ? (ke - kb + 63) / 64 : 0;
  const int s0 = (nst * wave) / NW, s1 = (nst * (wave + 1)) / NW;  // this wave's stages [s0, s1) of the split

  // Loads: lane l reads 16 B of row 8 i + l / 8 at chunk l % 8 of the stage's 128 B row, so every load covers
  // eight whole 128-byte lines (loads in the MFMA operand layout, 16 rows x 64 B each, streamed at about half the
  // rate). Rows past N (or M) read the last row instead (their outputs are never stored). Per-lane byte offsets of
  // the split's first stage; the stage part goes in soffset.
  const bool wpk = p.wpk != 0;
  const int nbw = p.N >> 4;
  const uint32_t wstride = wpk ? (uint32_t)nbw * 2048u : 128u;
  const int lrow = lane >> 3, lch = lane & 7;
  uint32_t wo[RW], xo[RX];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const int n = min(n0 + i * 8 + lrow, p.N - 1);
    wo[i] = wpk ? (uint32_t)((((kb >> 6) * nbw + (n >> 4)) * 16 + (n & 15)) * 128 + lch * 16)
                : (uint32_t)(((int64_t)(n - n0) * p.ldw + kb + lch * 8) * 2);
  }
#pragma unroll
  for (int i = 0; i < RX; ++i) {
    const int m = min(i * 8 + lrow, p.M - m0 - 1);  // row within the x descriptor
    xo[i] = (uint32_t)(((int64_t)m * p.ldx + kb + lch * 8) * 2);
  }
  const __amdgpu_buffer_rsrc_t rsW =
      wpk ? make_rsrc(p.W, (int64_t)p.N * p.K * 2)
          : make_rsrc(p.W + (int64_t)n0 * p.ldw, ((int64_t)(min(BN, p.N - n0) - 1) * p.ldw + p.K) * 2);
  const __amdgpu_buffer_rsrc_t rsX =
      make_rsrc(p.X + (int64_t)m0 * p.ldx, ((int64_t)(min(BM, p.M - m0) - 1) * p.ldx + p.K) * 2);

  // A ring of D stages of loads in registers (compiler-visible loads: the compiler places the vmcnt waits). A
  // stage past the wave's run re-reads the run's last stage (the split's first, for a wave without stages) and
  // skips its MFMAs, so every stage issues the same loads and none sits behind a branch.
  uint4 rw[D][RW], rx[D][RX];
  const int slast = max(s1 - 1, 0);
  auto load = [&](const int d, const int s) {
    const int sc = min(s, slast);
    const uint32_t sw = __builtin_amdgcn_readfirstlane((uint32_t)sc * wstride);
    const uint32_t sx = __builtin_amdgcn_readfirstlane((uint32_t)sc * 128u);
#pragma unroll
    for (int i = 0; i < RW; ++i)
      rw[d][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsW, wo[i], sw, 2));
#pragma unroll
    for (int i = 0; i < RX; ++i)
      rx[d][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsX, xo[i], sx, 0));
  };

  // The wave's own LDS region, one stage (no other wave touches it, so no barrier; a wave's LDS accesses run in
  // order, so the next stage's stores cannot overtake this stage's operand reads): rows of 128 B, W rows first,
  // 16-byte chunk c of row r stored at chunk c ^ ((r / 2) % 8), so that the MFMA-layout reads (16 rows at one
  // chunk) fall on distinct banks.
  uint8_t* const mine = lds + wave * SLOT;
  // byte offset of this lane's chunk of row 8 i + lrow (even i, then odd i: the swizzle takes the row's bits 1..3)
  const int wr_off[2] = {lrow * 128 + ((lch ^ ((lrow >> 1) & 7)) << 4),
                         (8 + lrow) * 128 + ((lch ^ (((8 + lrow) >> 1) & 7)) << 4)};
  auto stage_in = [&](const int d) {
#pragma unroll
    for (int i = 0; i < RW; ++i) *reinterpret_cast<uint4*>(mine + (i >> 1) * 2048 + wr_off[i & 1]) = rw[d][i];
#pragma unroll
    for (int i = 0; i < RX; ++i)
      *reinterpret_cast<uint4*>(mine + BN * 128 + (i >> 1) * 2048 + wr_off[i & 1]) = rx[d][i];
  };
  // MFMA operand of 16-row block j (W blocks first, then x) for k32 half h: lane reads row lr, chunk 4 h + lg
  auto operand = [&](const int j, const int h) {
    const int c = (4 * h + lg) ^ ((lr >> 1) & 7);
    return *reinterpret_cast<const bf16x8*>(mine + (j * 16 + lr) * 128 + c * 16);
  };

  f32x4 acc[FW][FM];
#pragma unroll
  for (int f = 0; f < FW; ++f)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) acc[f][fm] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nround = (s1 - s0 + D - 1) / D;
  // Scheduling barriers keep the loads of each stage together and in stage order, so the compiler's count of the
  // loads still in flight is the same at the loop head from both sides and its waits stay exact (vmcnt(N), not a
  // full drain at every round).
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load(d, s0 + d);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int rd = 0; rd < nround; ++rd) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      stage_in(d);
      __builtin_amdgcn_sched_barrier(0);
      load(d, s0 + (rd + 1) * D + d);
      __builtin_amdgcn_sched_barrier(0);
      if (s0 + rd * D + d < s1) {  // wave-uniform: a re-read stage past the run adds nothing
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          bf16x8 xf[FM];
#pragma unroll
          for (int fm = 0; fm < FM; ++fm) xf[fm] = operand(FW + fm, h);
#pragma unroll
          for (int f = 0; f < FW; ++f) {
            const bf16x8 wf = operand(f, h);
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
              acc[f][fm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, xf[fm], acc[f][fm], 0, 0, 0);
          }
        }
      }
    }
  }

  // the NW partial tiles meet in LDS (in place of the stage buffers, once every wave is done with its own); wave q
  // sums fragment q (and q + NW, ...) in wave order and stores it
  static_assert(NF * 1024 <= SLOT, "partial tile fits the wave's region");
  f32x4 (*red)[NF][64] = reinterpret_cast<f32x4 (*)[NF][64]>(lds);
  __syncthreads();
#pragma unroll
  for (int f = 0; f < FW; ++f)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) red[wave][f * FM + fm][lane] = acc[f][fm];
  __syncthreads();
  for (int q = wave; q < NF; q += NW) {
    f32x4 v = red[0][q][lane];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[w][q][lane];
    const int f = q / FM, fm = q % FM;
    const int n = n0 + f * 16 + lg * 4;
    const int m = m0 + fm * 16 + lr;
    store_tile(p, epi, z, m, n, lg, v);
  }
}

#define OJX_SW_INST(FW, FM, NW, D) template __global__ void gemm_sw_kernel<FW, FM, NW, D>(const GemmParams, const int);
OJX_SW_INST(1, 1, 8, 4)
OJX_SW_INST(1, 1, 16, 4)
OJX_SW_INST(2, 1, 8, 4)
OJX_SW_INST(2, 1, 16, 3)
OJX_SW_INST(4, 1, 8, 3)
OJX_SW_INST(1, 2, 16, 3)
OJX_SW_INST(2, 2, 8, 3)
OJX_SW_INST(1, 1, 4, 6)

}  // namespace ojx
