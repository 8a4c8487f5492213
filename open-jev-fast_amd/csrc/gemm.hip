// bf16 projection GEMM for gfx950 (MI355X): y[M,N] = x[M,K] . W[N,K]^T, fp32 accumulation on MFMA.
//
// Replaces the reference's cuBLASLt GEMM (src/lt.cpp:43-55 lt_matmul, called from _mm in src/fastmodel.py:168-175)
// and its split-K torch.bmm with fp32 output (src/fastmodel.py:158-166), with the epilogues that follow them fused
// into the store (SiLU.mul of src/kernels.cu:76-89 / 1304-1331, residual add of src/kernels.cu:1464-1475).
//
// Design (one template, many tile shapes; the per-shape choice lives in the plan table of api.hip):
//   * The MFMA "A" operand is a 16-row slab of W and the "B" operand a 16-row slab of x, so each lane's
//     accumulator holds 4 consecutive output columns n of one output row m: stores are 8 B (bf16) / 16 B (fp32)
//     per lane and a fused gate/up pair sits in one lane pair.
//   * v_mfma_f32_16x16x32_bf16: lane l feeds row (l % 16) and the 8 K values of group (l / 16). A and B use the
//     same lane->K mapping, so the dot product is complete whatever order the hardware sums the K values in.
//   * Workgroup tile BN (W rows) x BM (x rows) x BK, WN x WM waves; both operand tiles are staged
//     global -> registers -> LDS with two LDS buffers, so the loads of tile t+1 are in flight while tile t is
//     multiplied. LDS rows are padded by 16 B, which puts the 16 rows read by one ds_read_b128 on distinct banks.
//   * Split-K over gridDim: each split owns a contiguous K range and writes an fp32 partial plane; a second
//     pass (epilogue.hip) reduces the planes in ascending split order (deterministic) and applies the epilogue.
//   * XCD-aware block order: MI355X dispatches workgroup b to XCD (b mod 8). Blocks are renumbered so that each
//     XCD runs a contiguous range of logical tiles, and the M tiles that share one W tile are adjacent in that
//     range, so a W tile is fetched from HBM into that XCD's L2 once.
#include "gemm_common.h"

#include <type_traits>

namespace ojx {

// ------------------------------------------------------------------------------------------------ one launch
// Arrival counters of the one-launch split-K (ol_epilogue, gemm_common.h): zero when the library loads, and every
// call leaves the counters it used at zero again (the last arrival re-arms its counter). Calls of one-launch plans
// that run at the same time on one GPU (different streams) share them and race.
__device__ uint32_t g_ol_tiles[kOlMaxTiles];
__device__ uint32_t g_ol_blocks[kOlMaxBlocks];

// Device addresses of the counters on the current device (looked up once per device, with it current).
hipError_t ol_counters(uint32_t** tiles, uint32_t** blocks) {
  static uint32_t* cache[64][2];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  if (cache[dev][0] == nullptr) {
    void* t = nullptr;
    void* b = nullptr;
    if ((e = hipGetSymbolAddress(&t, HIP_SYMBOL(g_ol_tiles))) != hipSuccess) return e;
    if ((e = hipGetSymbolAddress(&b, HIP_SYMBOL(g_ol_blocks))) != hipSuccess) return e;
    if (t == nullptr || b == nullptr) return hipErrorInvalidSymbol;
    cache[dev][1] = static_cast<uint32_t*>(b);
    cache[dev][0] = static_cast<uint32_t*>(t);
  }
  *tiles = cache[dev][0];
  *blocks = cache[dev][1];
  return hipSuccess;
}

template <int BN, int BM, int BK, int WN, int WM>
__global__ void __launch_bounds__(64 * WN * WM) gemm_nt_kernel(const GemmParams p, const int epi) {
  constexpr int NT = 64 * WN * WM;
  constexpr int FN = BN / (16 * WN);
  constexpr int FM = BM / (16 * WM);
  static_assert(FN * 16 * WN == BN && FM * 16 * WM == BM, "tile must split into 16x16 fragments");
  static_assert(BK % 32 == 0, "BK must be a multiple of the MFMA K (32)");
  constexpr int LS = BK + 8;      // padded LDS row, bf16 elements
  constexpr int CPR = BK / 8;     // 16-byte chunks per tile row
  constexpr int W_CH = BN * CPR, X_CH = BM * CPR;
  constexpr int CW = (W_CH + NT - 1) / NT, CX = (X_CH + NT - 1) / NT;

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* sW = smem;               // [2][BN][LS]
  uint16_t* sX = smem + 2 * BN * LS; // [2][BM][LS]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (lets the compiler use SGPRs)
  const int wn = wave % WN, wm = wave / WN;
  const int lr = lane & 15, lg = lane >> 4;

  // XCD-aware renumbering (see header comment): logical id L, M tile fastest, then split, then N tile.
  const int G = gridDim.x, b = blockIdx.x;
  const int q = G >> 3, r = G & 7, xcd = b & 7;
  const int L = xcd * q + min(xcd, r) + (b >> 3);
  const int tm = L % p.tiles_m;
  const int t2 = L / p.tiles_m;
  const int z = t2 % p.splits;
  const int tn = t2 / p.splits;

  const int n0 = tn * BN, m0 = tm * BM;
  const int kb = z * p.kchunk;
  const int ke = min(p.K, kb + p.kchunk);
  const int nk = ke > kb ? (ke - kb + BK - 1) / BK : 0;

  // descriptors cover this tile's rows only: rows past N (or M) read zeros. A packed W ([K/64][N/16][16][64], see
  // ojx_pack_weight) goes through one descriptor over the whole buffer, rows past N skipped.
  const bool wpk = p.wpk != 0;
  const __amdgpu_buffer_rsrc_t rsW = wpk ? make_rsrc(p.W, (int64_t)p.N * p.K * 2)
                                         : make_rsrc(p.W + (int64_t)n0 * p.ldw, (int64_t)min(BN, p.N - n0) * p.ldw * 2);
  const __amdgpu_buffer_rsrc_t rsX = make_rsrc(p.X + (int64_t)m0 * p.ldx, (int64_t)min(BM, p.M - m0) * p.ldx * 2);
  const int nbw = p.N >> 4;
  uint4 rw[CW], rx[CX];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CW; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, col = (c % CPR) * 8;
      const bool ok = (W_CH % NT == 0 || c < W_CH) && k0 + col < ke;
      uint32_t o;
      bool okw = ok;
      if (wpk) {
        const int n = n0 + row, k = k0 + col;
        o = (uint32_t)(((((k >> 6) * nbw + (n >> 4)) * 16 + (n & 15)) * 64 + (k & 63)) * 2);
        okw = ok && n < p.N;
      } else {
        o = (uint32_t)(row * p.ldw + k0 + col) * 2u;
      }
      rw[i] = bload_nt(rsW, okw ? o : kOOB);
    }
#pragma unroll
    for (int i = 0; i < CX; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, col = (c % CPR) * 8;
      const bool ok = (X_CH % NT == 0 || c < X_CH) && k0 + col < ke;
      rx[i] = bload(rsX, ok ? (uint32_t)(row * p.ldx + k0 + col) * 2u : kOOB);
    }
  };
  auto lstore = [&](int buf) {
    uint16_t* w = sW + buf * BN * LS;
    uint16_t* x = sX + buf * BM * LS;
#pragma unroll
    for (int i = 0; i < CW; ++i) {
      const int c = tid + i * NT;
      if (W_CH % NT == 0 || c < W_CH) *reinterpret_cast<uint4*>(w + (c / CPR) * LS + (c % CPR) * 8) = rw[i];
    }
#pragma unroll
    for (int i = 0; i < CX; ++i) {
      const int c = tid + i * NT;
      if (X_CH % NT == 0 || c < X_CH) *reinterpret_cast<uint4*>(x + (c / CPR) * LS + (c % CPR) * 8) = rx[i];
    }
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (nk > 0) {
    gload(kb);
    lstore(0);
    lds_barrier();
  }
  for (int t = 0; t < nk; ++t) {
    const int buf = t & 1;
    if (t + 1 < nk) gload(kb + (t + 1) * BK);
    const uint16_t* w = sW + buf * BN * LS + (wn * FN * 16 + lr) * LS + lg * 8;
    const uint16_t* x = sX + buf * BM * LS + (wm * FM * 16 + lr) * LS + lg * 8;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      bf16x8 a[FN], bx[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) a[i] = *reinterpret_cast<const bf16x8*>(w + i * 16 * LS + kk);
#pragma unroll
      for (int j = 0; j < FM; ++j) bx[j] = *reinterpret_cast<const bf16x8*>(x + j * 16 * LS + kk);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bx[j], acc[i][j], 0, 0, 0);
    }
    if (t + 1 < nk) lstore(buf ^ 1);
    lds_barrier();
  }

  // ---------------------------------------------------------------------------------------------- epilogue
  // lane holds acc[i][j][e] = y[m][n + e], m = m0 + (wm*FM + j)*16 + lr, n = n0 + (wn*FN + i)*16 + 4*lg.
  if (p.one_launch) {
    const __amdgpu_buffer_rsrc_t rsP = make_rsrc(p.ol_parts, (int64_t)p.splits * p.M * p.N * 4);
    const int64_t zo = (int64_t)z * p.M * p.N;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int n = n0 + (wn * FN + i) * 16 + lg * 4;
        const int m = m0 + (wm * FM + j) * 16 + lr;
        if (m < p.M && n < p.N)
          __builtin_amdgcn_raw_buffer_store_b128(acc[i][j], rsP, (uint32_t)((zo + (int64_t)m * p.N + n) * 4), 0, kCoh);
      }
    ol_epilogue<BN, BM, NT>(p, epi, tn, tm, reinterpret_cast<float*>(smem));
    return;
  }
#pragma unroll
  for (int i = 0; i < FN; ++i) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int n = n0 + (wn * FN + i) * 16 + lg * 4;
      const int m = m0 + (wm * FM + j) * 16 + lr;
      store_tile(p, epi, z, m, n, lg, acc[i][j]);
    }
  }
}

// ------------------------------------------------------------------------------------------------ W-direct
// Weight-streaming variant. Each wave owns FN 16-row slabs of W and loads them from HBM straight into MFMA
// operand registers, D k-steps (of 32) ahead through a register ring; W never passes through LDS. The x tile
// (BM = 16 FM rows, shared by the NW waves of the workgroup) is staged global -> registers -> LDS in stages of
// BKX k, double-buffered, the next stage's loads in flight during the current stage. LDS traffic per MFMA is
// then one x fragment read per FN MFMAs, and the HBM stream (W) has D * FN * 1 KiB in flight per wave.
template <int FN, int FM, int NW, int D, int BKX>
__global__ void __launch_bounds__(64 * NW) gemm_wd_kernel(const GemmParams p, const int epi) {
  constexpr int NT = 64 * NW;
  constexpr int BN = NW * FN * 16, BM = FM * 16;
  constexpr int SPS = BKX / 32;  // k32 steps per x stage
  static_assert(BKX % 32 == 0 && (SPS % D == 0 || D % SPS == 0), "ring depth and x stage must nest");
  constexpr int LS = BKX + 8;
  constexpr int CPR = BKX / 8;
  constexpr int X_CH = BM * CPR;
  constexpr int CX = (X_CH + NT - 1) / NT;

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* sX = smem;  // [2][BM][LS]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (lets the compiler use SGPRs)
  const int lr = lane & 15, lg = lane >> 4;

  const int G = gridDim.x, b = blockIdx.x;
  const int q = G >> 3, r = G & 7, xcd = b & 7;
  const int L = xcd * q + min(xcd, r) + (b >> 3);
  const int tm = L % p.tiles_m;
  const int t2 = L / p.tiles_m;
  const int z = t2 % p.splits;
  const int tn = t2 / p.splits;

  const int n0 = tn * BN, m0 = tm * BM;
  const int kb = z * p.kchunk;
  const int ke = min(p.K, kb + p.kchunk);
  const int T = ke > kb ? (ke - kb + 31) / 32 : 0;   // k32 steps
  const int nst = (T + SPS - 1) / SPS;               // x stages

  // this lane's W rows (one per fragment) as byte offsets in the tile's descriptor, and its 8-element K group
  const __amdgpu_buffer_rsrc_t rsW = make_rsrc(p.W + (int64_t)n0 * p.ldw, (int64_t)min(BN, p.N - n0) * p.ldw * 2);
  const __amdgpu_buffer_rsrc_t rsX = make_rsrc(p.X + (int64_t)m0 * p.ldx, (int64_t)min(BM, p.M - m0) * p.ldx * 2);
  uint32_t woff[FN];
#pragma unroll
  for (int f = 0; f < FN; ++f) woff[f] = (uint32_t)(((wave * FN + f) * 16 + lr) * p.ldw + kb + lg * 8) * 2u;
  const int klim = ke - kb - lg * 8;  // step t is in range for this lane iff t * 32 < klim

  bf16x8 wr[D][FN];
  auto wload = [&](int slot, int t) {
    const bool kin = t * 32 < klim;
#pragma unroll
    for (int f = 0; f < FN; ++f)
      wr[slot][f] = __builtin_bit_cast(bf16x8, bload_nt(rsW, kin ? woff[f] + (uint32_t)t * 64u : kOOB));
  };

  uint4 rx[CX];
  auto xload = [&](int st) {
    const int k0 = kb + st * BKX;
#pragma unroll
    for (int i = 0; i < CX; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, col = (c % CPR) * 8;
      const bool ok = (X_CH % NT == 0 || c < X_CH) && k0 + col < ke;
      rx[i] = bload(rsX, ok ? (uint32_t)(row * p.ldx + k0 + col) * 2u : kOOB);
    }
  };
  auto xstore = [&](int buf) {
    uint16_t* x = sX + buf * BM * LS;
#pragma unroll
    for (int i = 0; i < CX; ++i) {
      const int c = tid + i * NT;
      if (X_CH % NT == 0 || c < X_CH) *reinterpret_cast<uint4*>(x + (c / CPR) * LS + (c % CPR) * 8) = rx[i];
    }
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Steps run in rounds of R = max(D, SPS) so that the ring slot (t % D) and the step within the x stage
  // (t % SPS) are compile-time constants; the step count is padded to whole rounds with zero loads.
  constexpr int R = D > SPS ? D : SPS;
  const int nround = (nst * SPS + R - 1) / R;
  const int nst_p = nround * (R / SPS);  // x stages including padding (their loads are out of range: zeros)
  if (nround > 0) {
#pragma unroll
    for (int d = 0; d < D; ++d) wload(d, d);
    xload(0);
    xstore(0);
    lds_barrier();
    if (nst_p > 1) xload(1);
  }
  for (int rd = 0; rd < nround; ++rd) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int t = rd * R + j;
      const int s = rd * (R / SPS) + j / SPS;
      const int jj = j % SPS;
      const uint16_t* xs = sX + (s & 1) * BM * LS + lr * LS + lg * 8 + jj * 32;
      bf16x8 xf[FM];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) xf[fm] = *reinterpret_cast<const bf16x8*>(xs + fm * 16 * LS);
#pragma unroll
      for (int f = 0; f < FN; ++f)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
          acc[f][fm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wr[j % D][f], xf[fm], acc[f][fm], 0, 0, 0);
      wload(j % D, t + D);
      if (jj == SPS - 1) {
        if (s + 1 < nst_p) xstore((s & 1) ^ 1);
        lds_barrier();
        if (s + 2 < nst_p) xload(s + 2);
      }
    }
  }

  // epilogue: lane holds acc[f][fm][e] = y[m][n + e]
#pragma unroll
  for (int f = 0; f < FN; ++f) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int n = n0 + (wave * FN + f) * 16 + lg * 4;
      const int m = m0 + fm * 16 + lr;
      store_tile(p, epi, z, m, n, lg, acc[f][fm]);
    }
  }
}



// ------------------------------------------------------------------------------------------------ W-direct 32x32
// v_mfma_f32_32x32x16_bf16 version of the weight-streaming design: each wave owns FN 32-row slabs of W, streamed
// from HBM into operand registers through a ring of DG load groups, and multiplies them against FM 32-row x
// fragments of the workgroup's x tile, which sits in LDS in stages of 64 k. WN x WM waves: waves with the same wn
// stream the same W rows (the second request hits in L1/L2) and split the x tile (WM * FM fragments, all of M when
// it fits), so W is fetched from HBM once per x tile and the LDS traffic is one 1 KiB x fragment per FN MFMAs.
//
// K order: the 16-k steps are taken in groups of G = 4. Within group u, lane group g = lane / 32 uses the
// 8-element k chunks 8u + 4g + s for steps s = 0..3, so each lane reads 4 consecutive chunks (64 B) of its W row
// in one go and a row's 128 B line is read whole by its two lanes. x fragments are read from LDS with the same
// chunk mapping, so every product pairs matching k.
//
// Output layout of a 32x32 fragment: lane l holds rows (W) n = 8 r + 4 (l / 32) + e, r = 0..3, e = 0..3, of
// column (x row) m = l % 32. A packed gate/up block of 8 rows therefore splits between lanes l and l ^ 32.
template <int FN, int FM, int WN, int WM, int DG>
__global__ void __launch_bounds__(64 * WN * WM) gemm_w32_kernel(const GemmParams p, const int epi) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  constexpr int G = 4;                      // k16 steps per W load group and per x stage (64 k)
  constexpr int NT = 64 * WN * WM;
  constexpr int BN = WN * FN * 32, BM = WM * FM * 32;
  constexpr int LS = 64 + 8;                // padded LDS row of one x stage (bf16)
  constexpr int X_CH = BM * 8;              // 16-byte chunks per x stage
  constexpr int CX = (X_CH + NT - 1) / NT;
  constexpr int LPS = CX + FN * G;          // global loads each stage issues (x stage s + 2, W refill)
  static_assert(DG >= 2 && DG % 2 == 0, "even ring depth: x register sets alternate with the stage parity");
  static_assert((DG - 1) * LPS < 64 && FN * G + LPS < 64, "wait counts must fit vmcnt");

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* sX = smem;  // [2][BM][LS]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  const int wn = wave % WN, wm = wave / WN;  // W slab group, x fragment group of this wave

  const int Gd = gridDim.x, b = blockIdx.x;
  const int q = Gd >> 3, r = Gd & 7, xcd = b & 7;
  const int L = xcd * q + min(xcd, r) + (b >> 3);
  const int tm = L % p.tiles_m;
  const int t2 = L / p.tiles_m;
  const int z = t2 % p.splits;
  const int tn = t2 / p.splits;
  const int n0 = tn * BN, m0 = tm * BM;
  const int kb = z * p.kchunk;
  const int ke = min(p.K, kb + p.kchunk);
  const int nst = ke > kb ? (ke - kb + 63) / 64 : 0;  // stages of 64 k (= W load groups)

  const u32x4 rsW = make_rsrc4(p.W + (int64_t)n0 * p.ldw, (int64_t)min(BN, p.N - n0) * p.ldw * 2);
  const u32x4 rsX = make_rsrc4(p.X + (int64_t)m0 * p.ldx, (int64_t)min(BM, p.M - m0) * p.ldx * 2);
  uint32_t woff[FN];
#pragma unroll
  for (int f = 0; f < FN; ++f) woff[f] = (uint32_t)(((wn * FN + f) * 32 + lr) * p.ldw + kb + lh * 32) * 2u;
  const int klim = ke - kb - lh * 32;  // chunk c of group u is in range for this lane iff u*64 + 8c < klim

  // All global loads of the main loop are issued from inline assembly and waited for explicitly (see bload_asm):
  // every stage issues the same loads in the same order (past the end they are out of range and read zeros), so
  // each wait count below is exact.
  u32x4 wr[DG][FN][G];
  auto wload = [&](int slot, int u) {
#pragma unroll
    for (int f = 0; f < FN; ++f)
#pragma unroll
      for (int c = 0; c < G; ++c) {
        const bool ok = u * 64 + c * 8 < klim;
        wr[slot][f][c] = bload_asm_nt(rsW, ok ? woff[f] + (uint32_t)(u * 128 + c * 16) : kOOB);
      }
  };
  u32x4 rx[2][CX];
  auto xload = [&](int set, int st) {
    const int k0 = kb + st * 64;
#pragma unroll
    for (int i = 0; i < CX; ++i) {
      const int c = tid + i * NT;
      const int row = c >> 3, col = (c & 7) * 8;
      const bool ok = (X_CH % NT == 0 || c < X_CH) && k0 + col < ke;
      rx[set][i] = bload_asm_agpr(rsX, ok ? (uint32_t)(row * p.ldx + k0 + col) * 2u : kOOB);
    }
  };
  // waits that also tie the awaited registers to the wait, so their consumers cannot move above it
#define OJX_WAIT_W(N, slot)                                                                                    \
  _Pragma("unroll") for (int f_ = 0; f_ < FN; ++f_)                                                         \
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(wr[slot][f_][0]), "+v"(wr[slot][f_][1]), "+v"(wr[slot][f_][2]),  \
                 "+v"(wr[slot][f_][3]) : "n"(N) : "memory")
#define OJX_WAIT_X(N, set)                                                                                     \
  do {                                                                                                         \
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");                                                   \
    _Pragma("unroll") for (int i_ = 0; i_ < CX; ++i_) asm volatile("" : "+a"(rx[set][i_]));                    \
  } while (0)
  auto xstore = [&](int set, int buf) {
    const uint32_t x = (uint32_t)reinterpret_cast<uintptr_t>(sX + buf * BM * LS);
#pragma unroll
    for (int i = 0; i < CX; ++i) {
      const int c = tid + i * NT;
      if (X_CH % NT == 0 || c < X_CH) {
        const uint32_t a = x + (uint32_t)(((c >> 3) * LS + (c & 7) * 8) * 2);
        asm volatile("ds_write_b128 %0, %1" ::"v"(a), "a"(rx[set][i]) : "memory");
      }
    }
  };

  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // x fragment of step cs (0..3) of a stage held in LDS buffer buf: lane group lh reads chunk 4 lh + cs
  auto xread = [&](bf16x8 (&xf)[FM], int buf, int cs) {
    const uint16_t* xs = sX + buf * BM * LS + (wm * FM * 32 + lr) * LS + (lh * 4 + cs) * 8;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) xf[fm] = *reinterpret_cast<const bf16x8*>(xs + fm * 32 * LS);
  };

  const int nround = (nst + DG - 1) / DG;  // stages run in rounds of DG: ring slots are compile-time
  const int nst_p = nround * DG;           // padded stages read zeros
  // Stage u of x lives in LDS buffer u & 1 and register set u & 1. It is loaded at the start of stage u - 3,
  // written to LDS after the mid-stage barrier of stage u - 2 (into the buffer stage u - 2 has finished reading)
  // and made visible by the barrier of stage u - 1, whose last step already prefetches its first fragments. The
  // one barrier per stage thus sits between MFMA steps 2 and 3, with MFMA work queued on both sides of it.
  // Every stage issues the same loads in the same order, x stage s + 3 then the W refill (group s + DG - 1 into the
  // slot stage s - 1 consumed), and the prologue ends with the same pair, so each wait count is one constant: no
  // stage-dependent branch around a wait. Loads complete in order for vmcnt, so the x wait is placed to let the
  // latest W refill stay in flight.
  bf16x8 xa[FM], xb[FM];
  if (nround > 0) {
    xload(0, 0);
    xload(1, 1);
#pragma unroll
    for (int d = 0; d < DG - 2; ++d) wload(d, d);
    OJX_WAIT_X(0, 0);
    OJX_WAIT_X(0, 1);
#pragma unroll
    for (int d = 0; d < DG - 2; ++d) { OJX_WAIT_W(0, d); }
    xstore(0, 0);
    xstore(1, 1);
    xload(0, 2);
    wload(DG - 2, DG - 2);  // in the place of a stage's refill, after its x set
    lds_barrier();
    xread(xa, 0, 0);
  }
  for (int rd = 0; rd < nround; ++rd) {
#pragma unroll
    for (int j = 0; j < DG; ++j) {
      const int s = rd * DG + j;  // stage = W group
      const int buf = s & 1;
      xload((j + 1) & 1, s + 3);
      wload((j + DG - 1) % DG, s + DG - 1);
      // W group s, issued at stage s - DG + 1 (group DG - 2 at the end of the prologue) and followed by DG - 1
      // whole stages (groups below DG - 2 were waited for in the prologue; the count then covers them trivially)
      OJX_WAIT_W((DG - 1) * LPS, j);
#pragma unroll
      for (int cs = 0; cs < G; ++cs) {
        bf16x8 (&cur)[FM] = (cs & 1) ? xb : xa;
        bf16x8 (&nxt)[FM] = (cs & 1) ? xa : xb;
        if (cs == G - 1) {
          // x stage s + 2 (register set j & 1, loaded at the start of stage s - 1 or at the end of the prologue,
          // followed by one refill and this stage's loads) goes into the buffer this stage has finished reading,
          // once every wave is past its reads
          OJX_WAIT_X(FN * G + LPS, j & 1);
          lds_barrier();
          xstore(j & 1, buf);
          // first fragments of stage s + 1, written during stage s - 1 and visible since the barrier above
          xread(nxt, buf ^ 1, 0);
        } else {
          // next step's fragments are read a whole step ahead of their MFMAs (the scheduling fences keep the
          // compiler from sinking each read next to its use, which would expose the LDS latency on every MFMA)
          xread(nxt, buf, cs + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int f = 0; f < FN; ++f)
            acc[f][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wr[j][f][cs]), cur[fm],
                                                                 acc[f][fm], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  wait_vmcnt<0>();  // padding loads still in flight

#pragma unroll
  for (int f = 0; f < FN; ++f)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const f32x4 v = {acc[f][fm][4 * rr], acc[f][fm][4 * rr + 1], acc[f][fm][4 * rr + 2], acc[f][fm][4 * rr + 3]};
        const f32x4 u = epi == EPI_SILU ? shfl4(v, 32) : v;
        const int n = n0 + (wn * FN + f) * 32 + 8 * rr + 4 * lh;
        const int m = m0 + (wm * FM + fm) * 32 + lr;
        if (epi == EPI_SILU) store_silu_pair(p, m, n, lh == 0, v, u);
        else store4(p, epi, z, m, n, true, v, v);
      }
#undef OJX_WAIT_W
#undef OJX_WAIT_X
}

// ------------------------------------------------------------------------------------------------ W-direct 32x32, x by DMA
// The 32x32 weight-streaming design of gemm_w32_kernel with x copied global -> LDS by the DMA path of buffer loads
// (buffer_load_dwordx4 ... lds): no staging registers, no LDS store instructions. That leaves the register room for
// FN = 2 slabs per wave (each x fragment read from LDS feeds FN MFMAs, and each x byte fetched serves BN W rows).
//
// x stage layout in LDS: BM rows of 64 k (128 B), unpadded. One DMA instruction fills 1 KiB = 8 rows, lane t
// writing row t / 8 at 16-byte position q = t % 8; it fetches the row's chunk c = q ^ sw(row), sw(r) = (r / 2) % 8,
// so a global row is still read as one whole 128 B line, and the fragment reads (32 rows, one chunk) spread over
// all banks.
__device__ __forceinline__ void dma16_asm(const u32x4& r, uint32_t lds_addr, uint32_t voff) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds_addr) : "memory");
}

template <int FN, int FM, int WN, int WM, int DG>
__global__ void __launch_bounds__(64 * WN * WM) gemm_w32d_kernel(const GemmParams p, const int epi) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  constexpr int G = 4;                       // k16 steps per W load group and per x stage (64 k)
  constexpr int NWV = WN * WM;
  constexpr int BN = WN * FN * 32, BM = WM * FM * 32;
  constexpr int XB = BM * 128;               // bytes of one x stage
  constexpr int CXD = BM / 8 / NWV;          // DMA instructions per wave per stage
  static_assert(BM % (8 * NWV) == 0, "x stage rows must split evenly over the waves");
  constexpr int LPS = FN * G + CXD;          // loads each stage issues (W refill, x stage s + 2)
  static_assert(DG >= 2, "ring depth");
  static_assert((DG - 1) * LPS < 64 && FN * G < 64, "wait counts must fit vmcnt");

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  const uint32_t sbase = (uint32_t)reinterpret_cast<uintptr_t>(smem);  // [2][BM][64] bf16, swizzled

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  const int wn = wave % WN, wm = wave / WN;

  const int Gd = gridDim.x, b = blockIdx.x;
  const int q = Gd >> 3, r = Gd & 7, xcd = b & 7;
  const int L = xcd * q + min(xcd, r) + (b >> 3);
  const int tm = L % p.tiles_m;
  const int t2 = L / p.tiles_m;
  const int z = t2 % p.splits;
  const int tn = t2 / p.splits;
  const int n0 = tn * BN, m0 = tm * BM;
  const int kb = z * p.kchunk;
  const int ke = min(p.K, kb + p.kchunk);
  const int nst = ke > kb ? (ke - kb + 63) / 64 : 0;

  const u32x4 rsW = make_rsrc4(p.W + (int64_t)n0 * p.ldw, (int64_t)min(BN, p.N - n0) * p.ldw * 2);
  const u32x4 rsX = make_rsrc4(p.X + (int64_t)m0 * p.ldx, (int64_t)min(BM, p.M - m0) * p.ldx * 2);
  uint32_t woff[FN];
#pragma unroll
  for (int f = 0; f < FN; ++f) woff[f] = (uint32_t)(((wn * FN + f) * 32 + lr) * p.ldw + kb + lh * 32) * 2u;
  const int klim = ke - kb - lh * 32;

  // DMA source offsets: instruction i of this wave fills rows 8 (wave + i NWV) .. + 8 of the stage. With NWV even
  // the swizzle sw(row) = (4 (wave + i NWV) + lane / 16) % 8 does not depend on i, so one chunk column and one
  // offset serve all of the wave's instructions (instruction i adds 8 NWV rows).
  static_assert(NWV % 2 == 0, "even wave count: one DMA column per lane");
  const int xcol = ((lane & 7) ^ ((4 * wave + (lane >> 4)) & 7)) * 8;
  const uint32_t xoff = (uint32_t)((8 * wave + (lane >> 3)) * p.ldx + kb + xcol) * 2u;
  const uint32_t xstep = (uint32_t)(8 * NWV * p.ldx) * 2u;
  u32x4 wr[DG][FN][G];
  auto wload = [&](int slot, int u) {
#pragma unroll
    for (int f = 0; f < FN; ++f)
#pragma unroll
      for (int c = 0; c < G; ++c) {
        const bool ok = u * 64 + c * 8 < klim;
        wr[slot][f][c] = bload_asm_nt(rsW, ok ? woff[f] + (uint32_t)(u * 128 + c * 16) : kOOB);
      }
  };
  auto xdma = [&](int buf, int st) {
    const bool ok = st * 64 + xcol < ke - kb;
    const uint32_t o = xoff + (uint32_t)(st * 128);
#pragma unroll
    for (int i = 0; i < CXD; ++i)
      dma16_asm(rsX, sbase + (uint32_t)(buf * XB + (wave + i * NWV) * 1024), ok ? o + i * xstep : kOOB);
  };
#define OJX_WAIT_W(N, slot)                                                                                    \
  _Pragma("unroll") for (int f_ = 0; f_ < FN; ++f_)                                                         \
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(wr[slot][f_][0]), "+v"(wr[slot][f_][1]), "+v"(wr[slot][f_][2]),  \
                 "+v"(wr[slot][f_][3]) : "n"(N) : "memory")

  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // fragment reads: row r = (wm FM + fm) 32 + lr, chunk c = 4 lh + cs at position c ^ sw(r); sw depends on lr only
  const int sw = (lr >> 1) & 7;
  const uint16_t* xrow = smem + (wm * FM * 32 + lr) * 64;
  auto xread = [&](bf16x8 (&xf)[FM], int buf, int cs) {
    const uint16_t* xs = xrow + buf * (XB / 2) + (((lh * 4 + cs) ^ sw) * 8);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) xf[fm] = *reinterpret_cast<const bf16x8*>(xs + fm * 32 * 64);
  };

  const int nround = (nst + DG - 1) / DG;
  // Schedule (stage s = W group s = x stage s, x stage u in LDS buffer u & 1): at the start of stage s the W slot
  // stage s - 1 used is refilled with group s + DG - 1; between MFMA steps 2 and 3 the wave waits for its DMA of
  // stage s + 1 (issued one stage earlier, followed only by this stage's refill), passes the barrier that makes all
  // of stage s + 1 visible and frees buffer s & 1, then DMAs stage s + 2 into that buffer and prefetches the first
  // fragments of stage s + 1.
  bf16x8 xa[FM], xb[FM];
  if (nround > 0) {
    xdma(0, 0);
    xdma(1, 1);
#pragma unroll
    for (int d = 0; d < DG - 1; ++d) wload(d, d);
    wait_vmcnt<0>();
#pragma unroll
    for (int d = 0; d < DG - 1; ++d) { OJX_WAIT_W(0, d); }
    lds_barrier();
    xread(xa, 0, 0);
  }
  for (int rd = 0; rd < nround; ++rd) {
#pragma unroll
    for (int j = 0; j < DG; ++j) {
      const int s = rd * DG + j;
      const int buf = s & 1;
      wload((j + DG - 1) % DG, s + DG - 1);
      // group s: issued at the start of stage s - DG + 1, followed by DG - 1 whole stages of loads less that
      // stage's own refill... counted exactly: that stage's DMA, DG - 2 full stages, this stage's refill
      OJX_WAIT_W((DG - 1) * LPS, j);
#pragma unroll
      for (int cs = 0; cs < G; ++cs) {
        bf16x8 (&cur)[FM] = (cs & 1) ? xb : xa;
        bf16x8 (&nxt)[FM] = (cs & 1) ? xa : xb;
        if (cs == G - 1) {
          asm volatile("s_waitcnt vmcnt(%0)" ::"n"(FN * G) : "memory");
          lds_barrier();
          xdma(buf, s + 2);
          xread(nxt, buf ^ 1, 0);
        } else {
          xread(nxt, buf, cs + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int f = 0; f < FN; ++f)
            acc[f][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wr[j][f][cs]), cur[fm],
                                                                 acc[f][fm], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  wait_vmcnt<0>();  // padding loads still in flight
  lds_barrier();    // and the last DMAs' writes, before the workgroup's LDS can be handed to another one

#pragma unroll
  for (int f = 0; f < FN; ++f)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const f32x4 v = {acc[f][fm][4 * rr], acc[f][fm][4 * rr + 1], acc[f][fm][4 * rr + 2], acc[f][fm][4 * rr + 3]};
        const f32x4 u = epi == EPI_SILU ? shfl4(v, 32) : v;
        const int n = n0 + (wn * FN + f) * 32 + 8 * rr + 4 * lh;
        const int m = m0 + (wm * FM + fm) * 32 + lr;
        if (epi == EPI_SILU) store_silu_pair(p, m, n, lh == 0, v, u);
        else store4(p, epi, z, m, n, true, v, v);
      }
#undef OJX_WAIT_W
}

// ------------------------------------------------------------------------------------------------ LDS-DMA
// Both operand tiles go global -> LDS directly (buffer_load ... lds): no staging registers, so an NS-stage ring
// of K tiles (64 k each) can be in flight within the 160 KB LDS. Each stage is its own static LDS array, which
// gives every array its own alias scope, so the compiler's wait-count pass does not drain the whole queue before
// reading a stage; the waits are explicit (vmcnt = loads of the younger stages still allowed in flight).
//
// Fragment-major LDS layout: a stage holds 16-row x 8-element blocks (256 B: row-major 16 B per row), ordered
// (16-row group, k chunk). One DMA instruction fills 4 consecutive blocks with 1 KiB in lane order, and the MFMA
// operand read of one 16-row fragment for one k32 step is the same 1 KiB read linearly: conflict-free both ways.
template <int WN, int WM, int FN, int FM, int NS>
__global__ void __launch_bounds__(64 * WN * WM) gemm_dma_kernel(const GemmParams p, const int epi) {
  constexpr int NW = WN * WM;
  constexpr int BN = WN * FN * 16, BM = WM * FM * 16;
  constexpr int IW = BN / 8, IX = BM / 8;   // 1 KiB DMA instructions per stage for W / x
  constexpr int IPW = (IW + IX) / NW;       // per wave per stage
  static_assert((IW + IX) % NW == 0, "DMA instructions must split evenly over the waves");
  static_assert(NS >= 2 && NS <= 4, "2..4 stages");
  constexpr int STB = (BN + BM) * 128;      // bytes per stage
  constexpr int ALLOW = (NS - 2) * IPW;     // DMA instructions of younger stages allowed in flight
  static_assert(ALLOW < 64, "vmcnt range");
  constexpr int WAIT = (ALLOW & 0xF) | ((ALLOW >> 4) << 14) | (0x7 << 4);  // vmcnt(ALLOW) lgkmcnt(0)

  __shared__ __attribute__((aligned(1024))) uint8_t st0[STB];
  __shared__ __attribute__((aligned(1024))) uint8_t st1[STB];
  __shared__ __attribute__((aligned(1024))) uint8_t st2[NS > 2 ? STB : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t st3[NS > 3 ? STB : 16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (lets the compiler use SGPRs)
  const int wn = wave % WN, wm = wave / WN;

  const int G = gridDim.x, b = blockIdx.x;
  const int q = G >> 3, r = G & 7, xcd = b & 7;
  const int L = xcd * q + min(xcd, r) + (b >> 3);
  const int tm = L % p.tiles_m;
  const int t2 = L / p.tiles_m;
  const int z = t2 % p.splits;
  const int tn = t2 / p.splits;
  const int n0 = tn * BN, m0 = tm * BM;
  const int kb = z * p.kchunk;
  const int ke = min(p.K, kb + p.kchunk);
  const int nst = ke > kb ? (ke - kb + 63) / 64 : 0;

  const __amdgpu_buffer_rsrc_t rsW = make_rsrc(p.W + (int64_t)n0 * p.ldw, (int64_t)min(BN, p.N - n0) * p.ldw * 2);
  const __amdgpu_buffer_rsrc_t rsX = make_rsrc(p.X + (int64_t)m0 * p.ldx, (int64_t)min(BM, p.M - m0) * p.ldx * 2);

  // per-lane byte offsets (without the stage's k0) of this wave's DMA instructions
  uint32_t voff[IPW];
  int kcol[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int j = wave + i * NW;  // instruction index within the stage (W first, then x)
    const bool isw = j < IW;
    const int jj = isw ? j : j - IW;
    const int blk = jj * 4 + (lane >> 4);
    const int row = (blk >> 3) * 16 + (lane & 15);
    kcol[i] = (blk & 7) * 8;
    voff[i] = (uint32_t)(row * (isw ? p.ldw : p.ldx) + kb + kcol[i]) * 2u;
  }
  auto issue = [&](uint8_t* dst, int st) {
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int j = wave + i * NW;
      const bool isw = j < IW;
      const int ldsoff = isw ? j * 1024 : BN * 128 + (j - IW) * 1024;
      const bool ok = st * 64 + kcol[i] < ke - kb;
      if (isw) dma16_nt(rsW, dst + ldsoff, ok ? voff[i] + (uint32_t)st * 128u : kOOB);
      else dma16(rsX, dst + ldsoff, ok ? voff[i] + (uint32_t)st * 128u : kOOB);
    }
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const uint8_t* cur) {
    const uint8_t* wb = cur + (wn * FN) * 2048 + lane * 16;
    const uint8_t* xb = cur + BN * 128 + (wm * FM) * 2048 + lane * 16;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8 a[FN], x[FM];
#pragma unroll
      for (int f = 0; f < FN; ++f) a[f] = *reinterpret_cast<const bf16x8*>(wb + f * 2048 + kk * 1024);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) x[fm] = *reinterpret_cast<const bf16x8*>(xb + fm * 2048 + kk * 1024);
#pragma unroll
      for (int f = 0; f < FN; ++f)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
          acc[f][fm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[f], x[fm], acc[f][fm], 0, 0, 0);
    }
  };
  auto barrier = [&]() {
    __builtin_amdgcn_s_waitcnt(WAIT);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // prologue: stages 0 .. NS-2 in flight (padded stages read zeros)
  issue(st0, 0);
  if (NS > 2) issue(st1, 1);
  if (NS > 3) issue(st2, 2);
  for (int s = 0; s < nst; s += NS) {
    // stage s lives in st0, s+1 in st1, ...; the stage issued at step s+i goes to the array stage s+i-1 used
    barrier();
    if (NS == 2) issue(st1, s + 1); else if (NS == 3) issue(st2, s + 2); else issue(st3, s + 3);
    compute(st0);
    if (s + 1 < nst) {
      barrier();
      if (NS == 2) issue(st0, s + 2); else if (NS == 3) issue(st0, s + 3); else issue(st0, s + 4);
      compute(st1);
    }
    if (NS > 2 && s + 2 < nst) {
      barrier();
      if (NS == 3) issue(st1, s + 4); else issue(st1, s + 5);
      compute(st2);
    }
    if (NS > 3 && s + 3 < nst) {
      barrier();
      issue(st2, s + 6);
      compute(st3);
    }
  }
  // drain the padded loads still in flight before the workgroup's LDS is reused
  __builtin_amdgcn_s_waitcnt(0x7 << 4);

#pragma unroll
  for (int f = 0; f < FN; ++f) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int n = n0 + (wn * FN + f) * 16 + (lane >> 4) * 4;
      const int m = m0 + (wm * FM + fm) * 16 + (lane & 15);
      store_tile(p, epi, z, m, n, lane >> 4, acc[f][fm]);
    }
  }
}

// ------------------------------------------------------------------------------------------------ registry
typedef void (*GemmFn)(const GemmParams, const int);

struct TileEntry {
  TileInfo info;
  GemmFn fn;
  GemmFn fixup = nullptr;  // persistent family: second pass over the split stream-K tiles
  // persistent family: second pass fused with the residual RMSNorm (one workgroup per output row)
  void (*fixup_norm)(const GemmParams, const float*, const int32_t*, float, uint16_t*) = nullptr;
};

#define OJX_TILE(BN, BM, BK, WN, WM)                                                                         \
  {{BN, BM, BK, WN, WM, 64 * WN * WM, 2 * (BN + BM) * (BK + 8) * 2, 0}, gemm_nt_kernel<BN, BM, BK, WN, WM>}
// LDS-DMA tiles: WN x WM waves of FN x FM fragments, NS stages of 64 k (static LDS)
#define OJX_DMA(WN, WM, FN, FM, NS)                                                                          \
  {{WN * FN * 16, WM * FM * 16, 64, WN, WM, 64 * WN * WM, 0, 2}, gemm_dma_kernel<WN, WM, FN, FM, NS>}
// W-direct 32x32 tiles: BN = WN*FN*32 W rows, BM = WM*FM*32 x rows, W ring of DG groups of 64 k, x stages of 64 k
#define OJX_W32D(FN, FM, WN, WM, DG)                                                                         \
  {{WN * FN * 32, WM * FM * 32, 64, WN, WM, 64 * WN * WM, 2 * (WM * FM * 32) * 128, 4},                      \
   gemm_w32d_kernel<FN, FM, WN, WM, DG>}
// Persistent stream-K tiles: BN = WN*FN*16 W rows, BM = WM*FM*16 x rows, 64-k stages, two or three LDS buffers
#define OJX_SK(FN, FM, WN, WM)                                                                               \
  {{WN * FN * 16, WM * FM * 16, 64, WN, WM, 64 * WN * WM, sk_lds(WN * FN * 16, WM * FM * 16), 5},          \
   gemm_sk_kernel<FN, FM, WN, WM>, gemm_sk_fixup_kernel<FN, FM, WN, WM>,                                   \
   gemm_sk_fixup_rmsnorm_kernel<FN, FM, WN, WM>}
// K-interleaved pair tiles: BN = 16 FW W rows, BM = 16 (4 FX + XE) x rows, 8 waves, 64-k stages, two LDS buffers
#define OJX_KX(FW, FX, XE)                                                                                   \
  {{16 * FW, 16 * (4 * FX + XE), 64, 4, 2, 512, (3 * 16 * FW + 2 * 16 * (4 * FX + XE)) * 128, 6},           \
   gemm_kx_kernel<FW, FX, XE>}
#define OJX_W32(FN, FM, WN, WM, DG)                                                                          \
  {{WN * FN * 32, WM * FM * 32, 64, WN, WM, 64 * WN * WM, 2 * (WM * FM * 32) * 72 * 2, 3},                   \
   gemm_w32_kernel<FN, FM, WN, WM, DG>}
// W-direct tiles: BN = NW*FN*16 W rows, BM = FM*16 x rows, x stage BKX, W ring depth D (k32 steps)
#define OJX_WD(FN, FM, NW, D, BKX)                                                                           \
  {{NW * FN * 16, FM * 16, BKX, NW, 1, 64 * NW, 2 * (FM * 16) * (BKX + 8) * 2, 1}, gemm_wd_kernel<FN, FM, NW, D, BKX>}

// Order is the tile id used by the plan table; append only (ids are stored in plan_table.inc).
static const TileEntry kTiles[] = {
    OJX_TILE(64, 16, 128, 4, 1),    // 0  skinny M, weight streaming
    OJX_TILE(128, 16, 128, 4, 1),   // 1
    OJX_TILE(64, 32, 128, 4, 1),    // 2
    OJX_TILE(128, 32, 128, 4, 1),   // 3
    OJX_TILE(128, 64, 64, 4, 1),    // 4
    OJX_TILE(64, 64, 128, 2, 2),    // 5
    OJX_TILE(128, 128, 64, 2, 2),   // 6
    OJX_TILE(256, 128, 64, 4, 2),   // 7
    OJX_TILE(128, 256, 64, 2, 4),   // 8
    OJX_TILE(256, 256, 64, 4, 2),   // 9
    OJX_TILE(128, 96, 64, 4, 2),    // 10 M = 288 = 3 x 96
    OJX_TILE(64, 288, 64, 2, 2),    // 11 M = 288 in one tile, W read once
    OJX_TILE(128, 288, 64, 2, 2),   // 12
    OJX_TILE(256, 96, 64, 4, 2),    // 13
    OJX_TILE(128, 144, 64, 2, 3),   // 14 M = 288 = 2 x 144
    OJX_TILE(64, 16, 256, 4, 1),    // 15 skinny M, deeper K
    OJX_WD(4, 1, 4, 8, 256),        // 16 W-direct 256 x 16
    OJX_WD(4, 2, 4, 8, 256),        // 17 256 x 32
    OJX_WD(4, 4, 4, 4, 128),        // 18 256 x 64
    OJX_WD(4, 6, 4, 4, 128),        // 19 256 x 96
    OJX_WD(4, 8, 4, 4, 128),        // 20 256 x 128
    OJX_WD(2, 9, 4, 4, 128),        // 21 128 x 144
    OJX_WD(4, 9, 4, 2, 64),         // 22 256 x 144
    OJX_WD(2, 18, 4, 2, 64),        // 23 128 x 288
    OJX_WD(2, 8, 4, 4, 128),        // 24 128 x 128
    OJX_WD(2, 4, 4, 8, 256),        // 25 128 x 64
    OJX_WD(2, 1, 4, 8, 256),        // 26 128 x 16
    OJX_WD(4, 3, 4, 4, 128),        // 27 256 x 48
    OJX_WD(2, 18, 4, 8, 64),        // 28 128 x 288, deep W ring
    OJX_WD(2, 18, 4, 12, 64),       // 29
    OJX_WD(4, 9, 4, 8, 64),         // 30 256 x 144
    OJX_WD(2, 9, 4, 16, 64),        // 31 128 x 144
    OJX_WD(4, 6, 4, 8, 64),         // 32 256 x 96
    OJX_WD(4, 4, 4, 8, 64),         // 33 256 x 64
    OJX_WD(2, 4, 4, 16, 64),        // 34 128 x 64
    OJX_WD(4, 1, 4, 16, 64),        // 35 256 x 16
    OJX_WD(2, 2, 4, 16, 64),        // 36 128 x 32
    OJX_DMA(2, 2, 4, 9, 3),         // 37 128 x 288
    OJX_DMA(2, 2, 4, 4, 4),         // 38 128 x 128
    OJX_DMA(2, 2, 6, 8, 2),         // 39 192 x 256
    OJX_DMA(2, 2, 4, 8, 3),         // 40 128 x 256
    OJX_DMA(2, 2, 8, 4, 3),         // 41 256 x 128
    OJX_DMA(2, 2, 4, 6, 3),         // 42 128 x 192
    OJX_DMA(2, 2, 2, 9, 3),         // 43 64 x 288
    OJX_DMA(2, 2, 4, 2, 4),         // 44 128 x 64
    OJX_DMA(2, 2, 4, 1, 4),         // 45 128 x 32
    OJX_DMA(2, 2, 2, 1, 4),         // 46 64 x 32
    OJX_DMA(2, 2, 4, 9, 2),         // 47 128 x 288, 2 stages
    OJX_W32(1, 9, 4, 1, 4),         // 48 128 x 288 (32x32 MFMA, all of M = 288 per tile)
    OJX_W32(1, 9, 4, 1, 2),         // 49
    OJX_W32(1, 4, 4, 1, 4),         // 50 128 x 128
    OJX_W32(2, 4, 4, 1, 2),         // 51 256 x 128
    OJX_W32(1, 2, 4, 1, 4),         // 52 128 x 64
    OJX_W32(2, 2, 4, 1, 4),         // 53 256 x 64
    OJX_W32(1, 1, 4, 1, 4),         // 54 128 x 32
    OJX_W32(2, 1, 4, 1, 4),         // 55 256 x 32
    OJX_W32(1, 6, 4, 1, 4),         // 56 128 x 192
    OJX_W32(1, 8, 4, 1, 4),         // 57 128 x 256
    OJX_W32(1, 3, 4, 1, 4),         // 58 128 x 96
    OJX_W32(1, 5, 4, 1, 4),         // 59 128 x 160
    OJX_W32(2, 5, 2, 2, 2),         // 60 128 x 320 (M = 288 + 1 padded fragment), x split over 2 waves
    OJX_W32(2, 4, 2, 2, 4),         // 61 128 x 256
    OJX_W32(2, 4, 2, 2, 2),         // 62 128 x 256
    OJX_W32(2, 3, 2, 2, 2),         // 63 128 x 192
    OJX_W32(2, 2, 2, 2, 4),         // 64 128 x 128
    OJX_W32(2, 1, 2, 2, 4),         // 65 128 x 64
    OJX_W32D(1, 9, 4, 1, 4),        // 66 128 x 288, x by DMA
    OJX_W32D(2, 3, 4, 1, 2),        // 67 256 x 96
    OJX_W32D(2, 8, 4, 1, 2),        // 68 256 x 256
    OJX_W32D(2, 6, 4, 1, 2),        // 69 256 x 192
    OJX_W32D(2, 4, 4, 1, 2),        // 70 256 x 128
    OJX_W32D(2, 5, 2, 2, 2),        // 71 128 x 320
    OJX_W32D(1, 9, 4, 1, 2),        // 72 128 x 288
    OJX_SK(8, 4, 2, 4),             // 73 256 x 256 persistent, stream-K remainder
    OJX_SK(4, 9, 4, 2),             // 74 256 x 288
    OJX_SK(4, 4, 4, 2),             // 75 256 x 128
    OJX_SK(4, 6, 4, 2),             // 76 256 x 192
    OJX_SK(4, 3, 4, 2),             // 77 256 x 96
    OJX_SK(2, 9, 4, 2),             // 78 128 x 288
    OJX_SK(3, 9, 4, 2),             // 79 192 x 288: 182 W tiles at M <= 288, one round on 256 CUs
    OJX_KX(9, 4, 2),                // 80 144 x 288 K-interleaved pairs: 242 W tiles of the gate-up at M <= 288
    OJX_KX(8, 4, 2),                // 81 128 x 288
    OJX_KX(9, 2, 1),                // 82 144 x 144
    OJX_KX(8, 4, 0),                // 83 128 x 256
    OJX_KX(9, 1, 0),                // 84 144 x 64: M <= 64, 242 W tiles of the gate-up
    OJX_KX(9, 2, 0),                // 85 144 x 128
    OJX_KX(8, 2, 0),                // 86 128 x 128
    OJX_KX(8, 1, 0),                // 87 128 x 64
    OJX_KX(16, 2, 0),               // 88 256 x 128: one 256-dim attention head per tile (prep epilogue)
    OJX_KX(16, 1, 0),               // 89 256 x 64
    OJX_TILE(32, 16, 128, 2, 1),    // 90 skinny M, 32 W rows: N / 32 workgroups without split-K
    OJX_TILE(32, 16, 256, 2, 1),    // 91 the same, deeper K stages
    OJX_KX(10, 4, 0),               // 92 160 x 256: N = 5120 in 32 W tiles, 256 tiles at M = 2048
    OJX_KX(10, 2, 0),               // 93 160 x 128: 256 tiles at M = 1024
};

static bool g_attr_set[sizeof(kTiles) / sizeof(kTiles[0])];

int num_tiles() { return (int)(sizeof(kTiles) / sizeof(kTiles[0])); }

const TileInfo* tile_info(int tile) {
  if (tile < 0 || tile >= num_tiles()) return nullptr;
  return &kTiles[tile].info;
}

static hipError_t set_attr(int tile) {
  if (g_attr_set[tile]) return hipSuccess;
  const TileEntry& e = kTiles[tile];
  if (e.info.lds_bytes == 0) {  // static LDS only
    g_attr_set[tile] = true;
    return hipSuccess;
  }
  hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(e.fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, e.info.lds_bytes);
  if (err == hipSuccess) g_attr_set[tile] = true;
  return err;
}

hipError_t init_tiles() {
  for (int t = 0; t < num_tiles(); ++t) {
    hipError_t err = set_attr(t);
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

static hipError_t launch_main(const TileEntry& e, int tile, int epi, const GemmParams& p, hipStream_t stream,
                              int grid) {
  hipError_t err = set_attr(tile);
  if (err != hipSuccess) return err;
  if (grid <= 0) grid = p.tiles_n * p.tiles_m * p.splits;
  hipLaunchKernelGGL(e.fn, dim3(grid), dim3(e.info.threads), e.info.lds_bytes, stream, p, epi);
  return hipGetLastError();
}

hipError_t launch_gemm_residual_rmsnorm_sk(int tile, const GemmParams& p, const float* w1, const int32_t* rowmask,
                                           float eps, uint16_t* hn_out, hipStream_t stream, int grid) {
  const TileEntry& e = kTiles[tile];
  if (e.fixup_norm == nullptr || p.sk_ws == nullptr || p.N % 8 != 0 || p.N / 8 > 1024) return hipErrorInvalidValue;
  hipError_t err = launch_main(e, tile, EPI_RESID, p, stream, grid);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(e.fixup_norm, dim3(p.M), dim3(p.N / 8), 0, stream, p, w1, rowmask, eps, hn_out);
  return hipGetLastError();
}

hipError_t launch_gemm(int tile, int epi, const GemmParams& p, hipStream_t stream, int grid) {
  const TileEntry& e = kTiles[tile];
  hipError_t err = launch_main(e, tile, epi, p, stream, grid);
  if (err != hipSuccess || e.fixup == nullptr || p.sk_ws == nullptr) return err;
  const int rem = p.tiles_n * p.tiles_m - p.dp_tiles;  // the stream-K tiles
  hipLaunchKernelGGL(e.fixup, dim3(rem * (e.info.bm / 16)), dim3(256), 0, stream, p, epi);  // per 16-row block
  return hipGetLastError();
}

}  // namespace ojx
