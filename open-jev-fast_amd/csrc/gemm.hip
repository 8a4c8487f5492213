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
#include "ojx_internal.h"

namespace ojx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

  uint4 rw[CW], rx[CX];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CW; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, col = (c % CPR) * 8;
      const int n = n0 + row, k = k0 + col;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if ((W_CH % NT == 0 || c < W_CH) && n < p.N && k < ke)
        v = *reinterpret_cast<const uint4*>(p.W + (int64_t)n * p.ldw + k);
      rw[i] = v;
    }
#pragma unroll
    for (int i = 0; i < CX; ++i) {
      const int c = tid + i * NT;
      const int row = c / CPR, col = (c % CPR) * 8;
      const int m = m0 + row, k = k0 + col;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if ((X_CH % NT == 0 || c < X_CH) && m < p.M && k < ke)
        v = *reinterpret_cast<const uint4*>(p.X + (int64_t)m * p.ldx + k);
      rx[i] = v;
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
    __syncthreads();
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
    __syncthreads();
  }

  // ---------------------------------------------------------------------------------------------- epilogue
  // lane holds acc[i][j][e] = y[m][n + e], m = m0 + (wm*FM + j)*16 + lr, n = n0 + (wn*FN + i)*16 + 4*lg.
#pragma unroll
  for (int i = 0; i < FN; ++i) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int n = n0 + (wn * FN + i) * 16 + lg * 4;
      const int m = m0 + (wm * FM + j) * 16 + lr;
      const f32x4 v = acc[i][j];
      if (epi == EPI_SILU) {
        // Packed W_gu rows come in blocks of 8: 4 gate rows then the 4 up rows of the same columns, so lane
        // group lg (even) holds gate columns and lane group lg+1 the matching up columns.
        const float u0 = __shfl_xor(v[0], 16), u1 = __shfl_xor(v[1], 16);
        const float u2 = __shfl_xor(v[2], 16), u3 = __shfl_xor(v[3], 16);
        if ((lg & 1) == 0 && m < p.M && n < p.N) {
          const float g[4] = {v[0], v[1], v[2], v[3]};
          const float u[4] = {u0, u1, u2, u3};
          uint32_t o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = f2bf(rbf(silu_f(rbf(g[e]))) * rbf(u[e]));
          uint16_t* dst = reinterpret_cast<uint16_t*>(p.out) + (int64_t)m * p.ldo + (n >> 1);
          *reinterpret_cast<uint2*>(dst) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
        }
      } else if (m < p.M && n < p.N) {
        if (epi == EPI_F32) {
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
    }
  }
}

// ------------------------------------------------------------------------------------------------ registry
typedef void (*GemmFn)(const GemmParams, const int);

struct TileEntry {
  TileInfo info;
  GemmFn fn;
};

#define OJX_TILE(BN, BM, BK, WN, WM)                                                                         \
  {{BN, BM, BK, WN, WM, 64 * WN * WM, 2 * (BN + BM) * (BK + 8) * 2}, gemm_nt_kernel<BN, BM, BK, WN, WM>}

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

hipError_t launch_gemm(int tile, int epi, const GemmParams& p, hipStream_t stream) {
  const TileEntry& e = kTiles[tile];
  hipError_t err = set_attr(tile);
  if (err != hipSuccess) return err;
  const int grid = p.tiles_n * p.tiles_m * p.splits;
  hipLaunchKernelGGL(e.fn, dim3(grid), dim3(e.info.threads), e.info.lds_bytes, stream, p, epi);
  return hipGetLastError();
}

}  // namespace ojx
