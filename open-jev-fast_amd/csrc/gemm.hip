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

#include <atomic>
#include <mutex>
#include <type_traits>

namespace ojx {

// ------------------------------------------------------------------------------------------------ one launch
// Arrival counters of the one-launch split-K (ol_epilogue, gemm_common.h): zero when the library loads, and every
// call leaves the counters it used at zero again (the last arrival re-arms its counter). There are kOlSets sets per
// device; each stream that launches a one-launch plan is given a set of its own, the first time it does, so calls
// on different streams (each with its own workspace) may overlap. Streams beyond kOlSets on one device share sets
// (chosen by the stream's handle), and calls that overlap on a shared set race; so do graph replays on a stream
// other than the one they were captured on, which keep the capture stream's set.
__device__ uint32_t g_ol_tiles[kOlSets * kOlMaxTiles];
__device__ uint32_t g_ol_blocks[kOlSets * kOlMaxBlocks];

// Device addresses of the counters of `stream`'s set on the current device (the symbol looked up once per device,
// with it current).
hipError_t ol_counters(hipStream_t stream, uint32_t** tiles, uint32_t** blocks) {
  constexpr int kDev = 64;
  static std::mutex mu;
  static uint32_t* base[kDev][2];
  static hipStream_t owner[kDev][kOlSets];
  static int owners[kDev];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kDev) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (base[dev][0] == nullptr) {
    void* t = nullptr;
    void* b = nullptr;
    if ((e = hipGetSymbolAddress(&t, HIP_SYMBOL(g_ol_tiles))) != hipSuccess) return e;
    if ((e = hipGetSymbolAddress(&b, HIP_SYMBOL(g_ol_blocks))) != hipSuccess) return e;
    if (t == nullptr || b == nullptr) return hipErrorInvalidSymbol;
    base[dev][1] = static_cast<uint32_t*>(b);
    base[dev][0] = static_cast<uint32_t*>(t);
  }
  int set = -1;
  for (int i = 0; i < owners[dev] && set < 0; ++i)
    if (owner[dev][i] == stream) set = i;
  if (set < 0 && owners[dev] < kOlSets) {
    set = owners[dev]++;
    owner[dev][set] = stream;
  }
  if (set < 0) set = (int)((reinterpret_cast<uintptr_t>(stream) >> 4) % kOlSets);
  *tiles = base[dev][0] + (size_t)set * kOlMaxTiles;
  *blocks = base[dev][1] + (size_t)set * kOlMaxBlocks;
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
// Persistent stream-K tiles: BN = WN*FN*16 W rows, BM = WM*FM*16 x rows, 64-k stages, two or three LDS buffers
#define OJX_SK(FN, FM, WN, WM)                                                                               \
  {{WN * FN * 16, WM * FM * 16, 64, WN, WM, 64 * WN * WM, sk_lds(WN * FN * 16, WM * FM * 16), 5},          \
   gemm_sk_kernel<FN, FM, WN, WM>, gemm_sk_fixup_kernel<FN, FM, WN, WM>,                                   \
   gemm_sk_fixup_rmsnorm_kernel<FN, FM, WN, WM>}
// Retired ids (16-72: register-streamed W, LDS-DMA and 32x32-MFMA tiles, slower than families 0, 5 and 6 on every
// measured shape): kept so that stored ids keep their meaning; nothing plans, fits or launches them.
#define OJX_RETIRED {{0, 0, 0, 0, 0, 0, 0, -1}, nullptr}
// K-interleaved pair tiles: BN = 16 FW W rows, BM = 16 (4 FX + XE) x rows, 8 waves, 64-k stages; an x ring of XD
// stages (the prefetch distance) and a W ring of XD + 1
#define OJX_KXD(FW, FX, XE, XD)                                                                              \
  {{16 * FW, 16 * (4 * FX + XE), 64, 4, 2, 512, ((XD + 1) * 16 * FW + XD * 16 * (4 * FX + XE)) * 128, 6},   \
   gemm_kx_kernel<FW, FX, XE, XD>}
#define OJX_KX(FW, FX, XE) OJX_KXD(FW, FX, XE, 2)

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
    OJX_RETIRED,                    // 16
    OJX_RETIRED,                    // 17
    OJX_RETIRED,                    // 18
    OJX_RETIRED,                    // 19
    OJX_RETIRED,                    // 20
    OJX_RETIRED,                    // 21
    OJX_RETIRED,                    // 22
    OJX_RETIRED,                    // 23
    OJX_RETIRED,                    // 24
    OJX_RETIRED,                    // 25
    OJX_RETIRED,                    // 26
    OJX_RETIRED,                    // 27
    OJX_RETIRED,                    // 28
    OJX_RETIRED,                    // 29
    OJX_RETIRED,                    // 30
    OJX_RETIRED,                    // 31
    OJX_RETIRED,                    // 32
    OJX_RETIRED,                    // 33
    OJX_RETIRED,                    // 34
    OJX_RETIRED,                    // 35
    OJX_RETIRED,                    // 36
    OJX_RETIRED,                    // 37
    OJX_RETIRED,                    // 38
    OJX_RETIRED,                    // 39
    OJX_RETIRED,                    // 40
    OJX_RETIRED,                    // 41
    OJX_RETIRED,                    // 42
    OJX_RETIRED,                    // 43
    OJX_RETIRED,                    // 44
    OJX_RETIRED,                    // 45
    OJX_RETIRED,                    // 46
    OJX_RETIRED,                    // 47
    OJX_RETIRED,                    // 48
    OJX_RETIRED,                    // 49
    OJX_RETIRED,                    // 50
    OJX_RETIRED,                    // 51
    OJX_RETIRED,                    // 52
    OJX_RETIRED,                    // 53
    OJX_RETIRED,                    // 54
    OJX_RETIRED,                    // 55
    OJX_RETIRED,                    // 56
    OJX_RETIRED,                    // 57
    OJX_RETIRED,                    // 58
    OJX_RETIRED,                    // 59
    OJX_RETIRED,                    // 60
    OJX_RETIRED,                    // 61
    OJX_RETIRED,                    // 62
    OJX_RETIRED,                    // 63
    OJX_RETIRED,                    // 64
    OJX_RETIRED,                    // 65
    OJX_RETIRED,                    // 66
    OJX_RETIRED,                    // 67
    OJX_RETIRED,                    // 68
    OJX_RETIRED,                    // 69
    OJX_RETIRED,                    // 70
    OJX_RETIRED,                    // 71
    OJX_RETIRED,                    // 72
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
    OJX_KXD(8, 1, 0, 4),            // 94 128 x 64, DMAs 4 stages ahead (weight streaming at M = 64-128)
};

// Per device (the attribute is set with the device current) and per tile; threads that race here both set the same
// attribute, which is harmless.
constexpr int kAttrDevices = 64;
static std::atomic<bool> g_attr_set[kAttrDevices][sizeof(kTiles) / sizeof(kTiles[0])];

int num_tiles() { return (int)(sizeof(kTiles) / sizeof(kTiles[0])); }

const TileInfo* tile_info(int tile) {
  if (tile < 0 || tile >= num_tiles()) return nullptr;
  return &kTiles[tile].info;
}

static hipError_t set_attr(int tile) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev < 0 || dev >= kAttrDevices) return hipErrorInvalidDevice;
  std::atomic<bool>& done = g_attr_set[dev][tile];
  if (done.load(std::memory_order_acquire)) return hipSuccess;
  const TileEntry& e = kTiles[tile];
  if (e.fn != nullptr && e.info.lds_bytes != 0)  // not a retired id, and dynamic LDS
    err = hipFuncSetAttribute(reinterpret_cast<const void*>(e.fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                              e.info.lds_bytes);
  if (err == hipSuccess) done.store(true, std::memory_order_release);
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
  if (tile < 0 || tile >= num_tiles()) return hipErrorInvalidValue;
  const TileEntry& e = kTiles[tile];
  if (e.fixup_norm == nullptr || p.sk_ws == nullptr || p.N % 8 != 0 || p.N / 8 > 1024) return hipErrorInvalidValue;
  hipError_t err = launch_main(e, tile, EPI_RESID, p, stream, grid);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(e.fixup_norm, dim3(p.M), dim3(p.N / 8), 0, stream, p, w1, rowmask, eps, hn_out);
  return hipGetLastError();
}

hipError_t launch_gemm(int tile, int epi, const GemmParams& p, hipStream_t stream, int grid) {
  if (tile < 0 || tile >= num_tiles() || kTiles[tile].fn == nullptr) return hipErrorInvalidValue;  // retired id
  const TileEntry& e = kTiles[tile];
  hipError_t err = launch_main(e, tile, epi, p, stream, grid);
  if (err != hipSuccess || e.fixup == nullptr || p.sk_ws == nullptr) return err;
  const int rem = p.tiles_n * p.tiles_m - p.dp_tiles;  // the stream-K tiles
  hipLaunchKernelGGL(e.fixup, dim3(rem * (e.info.bm / 16)), dim3(256), 0, stream, p, epi);  // per 16-row block
  return hipGetLastError();
}

}  // namespace ojx
