// Internal declarations shared by the HIP translation units of libojx (not part of the C-ABI).
//
// Conventions used throughout:
//   * bf16 values travel as raw 16-bit patterns (uint16_t); conversions are explicit and round to nearest even,
//     which is what torch's c10::BFloat16 and CUDA's __float2bfloat16 do (reference: src/kernels.cu:12-13).
//   * A projection computes y[M,N] = x[M,K] . W[N,K]^T with both operands K-contiguous ("NT"), the layout of
//     the reference's lt_matmul (src/lt.cpp:22-29) and F.linear.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ojx {

// ----------------------------------------------------------------------------------------------------------------
// bf16 helpers
__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
// fp32 -> bf16 bits, round to nearest, ties to even (NaN stays NaN): one v_cvt_pk_bf16_f32 on gfx950, in place
// of the five integer operations of the same rounding written out. The epilogues round three times per SiLU.mul
// output, and on the persistent kernel that arithmetic is VALU-throughput bound.
__device__ __forceinline__ uint32_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }  // round through bf16
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ uint32_t pack2(float a, float b) { return f2bf(a) | (f2bf(b) << 16); }

// Sum over the whole workgroup (wave64 butterfly, then one value per wave through LDS).
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

// RMSNorm of one row held by one workgroup of H/8 threads, 8 consecutive elements v[] per thread (the bf16-rounded
// h as floats): hn = bf16((h * rsqrt(sum h^2 / H + eps)) * w1), zero on a masked row (reference: add_rmsnorm_k,
// src/kernels.cu:41-73). Each thread sums its own 8 squares in order, then block_sum: every kernel that normalises
// a row this way gets the same bits.
__device__ __forceinline__ void rmsnorm_row8(const float (&v)[8], float4 wa, float4 wb, bool keep, float eps, int H,
                                             float* red, uint16_t* hn_dst) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += v[j] * v[j];
  ss = block_sum(ss, red);
  const float r = rsqrtf(ss / (float)H + eps);
  const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = keep ? (v[j] * r) * wv[j] : 0.f;
  *reinterpret_cast<uint4*>(hn_dst) =
      make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]), pack2(o[6], o[7]));
}

// ----------------------------------------------------------------------------------------------------------------
// GEMM epilogue modes (what a workgroup does with its fp32 accumulator tile)
enum Epi : int {
  EPI_BF16 = 0,   // y = bf16(acc)
  EPI_F32 = 1,    // split-K partial: parts[z][m][n] = acc (fp32)
  EPI_RESID = 2,  // h = bf16(residual + bf16(acc))
  EPI_SILU = 3,   // packed gate/up rows -> out = bf16(bf16(silu(bf16 g)) * bf16 u)
  EPI_FATTN = 4,  // full-attention QKV in-projection with the attention prep (K-interleaved 256-row tiles only)
  EPI_COUNT = 5
};

// Operands of the full-attention prep epilogue (see fullattn_prep_k in prep.hip for the arithmetic).
struct FattnParams {
  const float* qw1; const float* kw1;     // [D] fp32 RMSNorm weights (1 + weight) of q and k heads
  const uint16_t* cosb; const uint16_t* sinb;  // [M, RD] bf16
  uint16_t* qt; uint16_t* kt; uint16_t* vt;    // [HQ, M, D], [HKV, M, D], [HKV, M, D]
  uint16_t* gate;                              // [M, HQ D]
  int HQ, HKV, RD;
  float eps;
};

struct GemmParams {
  const uint16_t* W; int64_t ldw;   // [N, K] bf16, row stride ldw elements
  const uint16_t* X; int64_t ldx;   // [M, K] bf16, row stride ldx elements
  void* out; int64_t ldo;           // bf16 [M, N] (or [M, N/2] for EPI_SILU), or fp32 parts [S, M, N]
  const uint16_t* res; int64_t ldr; // residual [M, N] bf16 for EPI_RESID
  int64_t part_stride;              // elements between split-K partial planes (EPI_F32)
  int M, N, K;
  int kchunk;                       // K elements per split (multiple of 8; the last split may be shorter)
  int tiles_n, tiles_m, splits;
  // persistent stream-K kernels (family 5) only
  float* sk_ws;                     // partial-tile slots, 2 per workgroup, BN*BM fp32 each
  int dp_tiles;                     // tiles done whole first (a multiple of the grid)
  int wpk;                          // 1: W is in the stage-major packed layout (see ojx_pack_weight)
  FattnParams fa;                   // EPI_FATTN only
  int sk_grid;                      // workgroups that share the remaining tiles' K iterations
  // one-launch split-K (family 0, splits > 1): the fp32 planes, the split reduction with its epilogue and, for the
  // residual epilogue with hn, the rows' RMSNorm all run in the GEMM launch (see ol_epilogue in gemm.hip)
  int one_launch;                   // 1: reduction in the launch; 2: and the residual epilogue's RMSNorm (hn)
  uint32_t* ol_tiles; uint32_t* ol_blocks;  // the stream's set of the library's arrival counters (ol_counters)
  float* ol_parts;                  // [S, M, N] fp32 planes (workspace)
  float* ol_ss;                     // [tiles_n, M] fp32 sums of h^2 over each N tile's columns (workspace)
  const float* w1; const int32_t* rowmask; float eps;
  uint16_t* hn;                     // RMSNorm output [M, N] of the residual epilogue (null: h only)
};

// Arrival counters of the one-launch split-K (gemm.hip): per tile and per M block of a launch, in kOlSets sets per
// device, one per stream (streams beyond kOlSets share).
constexpr int kOlMaxTiles = 16384, kOlMaxBlocks = 4096, kOlSets = 8;
hipError_t ol_counters(hipStream_t stream, uint32_t** tiles, uint32_t** blocks);

struct TileInfo {
  int bn, bm, bk, wn, wm;  // W rows, X rows, K depth, waves along N, waves along M
  int threads;
  int lds_bytes;
  int family;  // 0: both operands through LDS; 5: persistent, 2 waves per SIMD, whole-tile waves then stream-K
               // over the remainder; 6: K-interleaved wave pairs (both waves of a SIMD own the same fragments,
               // alternate 32-k halves); -1: a retired id (1-4 were W-direct, LDS-DMA and 32x32-MFMA tiles)
};

// Tile registry (gemm.hip)
int num_tiles();
hipError_t init_tiles();  // sets the dynamic-LDS limit of every tile kernel
const TileInfo* tile_info(int tile);
// grid: workgroups to launch; 0 = one per (tile, split) (the persistent family passes its own)
hipError_t launch_gemm(int tile, int epi, const GemmParams& p, hipStream_t stream, int grid = 0);
// Persistent family with a residual epilogue and split tiles: the GEMM (without its split-tile pass), then one
// launch per output row that sums the split tiles' pieces, adds the residual (h) and normalises the row (hn).
hipError_t launch_gemm_residual_rmsnorm_sk(int tile, const GemmParams& p, const float* w1, const int32_t* rowmask,
                                           float eps, uint16_t* hn_out, hipStream_t stream, int grid);

// Row / elementwise kernels (epilogue.hip)
hipError_t launch_reduce_bf16(const float* parts, int S, int64_t part_stride, uint16_t* y, int64_t ldy,
                              int M, int N, hipStream_t st);
hipError_t launch_reduce_silu(const float* parts, int S, int64_t part_stride, uint16_t* out, int64_t ldo,
                              int M, int N, hipStream_t st);
hipError_t launch_add_rmsnorm(const uint16_t* x, const uint16_t* delta_bf16, const float* parts, int S,
                              int64_t part_stride, const float* w1, const int32_t* rowmask, float eps,
                              uint16_t* h_out, uint16_t* hn_out, int M, int H, hipStream_t st);
hipError_t launch_silu_mul(const uint16_t* gu, const uint16_t* tab, uint16_t* out, int M, int I, hipStream_t st);
hipError_t launch_act_tables(uint16_t* silu_b, float* sig_f, hipStream_t st);
hipError_t launch_head_gemv(const uint16_t* hn, int64_t rows, const int64_t* lastidx, int64_t R, const float* w,
                            const float* bias, float* scores, int H, hipStream_t st);
hipError_t launch_pack_gate_up(const uint16_t* gate, const uint16_t* up, uint16_t* packed, int I, int K,
                               hipStream_t st);
// Full-attention prep from the in-projection output proj [N, (2 HQ + 2 HKV) D], D = 256 (prep.hip).
hipError_t launch_fullattn_prep(const uint16_t* proj, int64_t N, int HQ, int HKV, int RD, float eps,
                                const float* qw1, const float* kw1, const uint16_t* cosb, const uint16_t* sinb,
                                uint16_t* qt, uint16_t* kt, uint16_t* vt, uint16_t* gate, hipStream_t st);
hipError_t launch_linattn_prep(const uint16_t* proj, const int32_t* hist, const int32_t* rep_ptr,
                               const int32_t* rep_pos, int64_t N, int64_t R, const uint16_t* convw,
                               const uint16_t* A_log, const uint16_t* dt_bias, int KD, int VD, int HV, int RQ,
                               uint16_t* q, uint16_t* k, uint16_t* v, float* g, uint16_t* beta, hipStream_t st);
// W [N, K] row-major -> packed [K/64][N/16][16][64]: the 16-row x 64-k blocks of one 64-k stage of all rows are
// contiguous, so a tile's weights for one stage are one contiguous run (N % 16 == 0, K % 64 == 0).
hipError_t launch_pack_weight(const uint16_t* w, uint16_t* wp, int64_t N, int64_t K, hipStream_t st);
hipError_t launch_unsplit_weight(const uint16_t* wt, uint16_t* w, int64_t K, int64_t N, hipStream_t st);

}  // namespace ojx
