// Persistent bf16 projection GEMM for gfx950 with a stream-K remainder: y[M,N] = x[M,K] . W[N,K]^T, fp32
// accumulation on v_mfma_f32_16x16x32_bf16, epilogues fused into the store (same modes as gemm.hip).
//
// Replaces the reference's cuBLASLt GEMM (src/lt.cpp:43-55, called through _mm, src/fastmodel.py:168-175) and its
// split-K bmm (src/fastmodel.py:158-166) at the M where the projection stops being a pure weight stream.
//
// Why this shape of kernel:
//   * Eight waves per workgroup, two per SIMD, each owning a (FN x 16) x (FM x 16) block of the output: while
//     one wave waits on LDS or a barrier the other keeps the SIMD's MFMA pipe busy. The wave tiles are large
//     (64x144, 128x64, ...) so that LDS operand traffic stays near 90 B/clk per CU, about half of what the
//     LDS delivers on this part.
//   * Both operand tiles go global -> LDS by DMA (buffer_load ... lds, 16 B per lane, one 8-row x 128 B block per
//     wave instruction) in stages of 64 k, three LDS buffers where they fit (stages t+1 and t+2 in flight while
//     stage t is multiplied, so a wave's DMA queue does not drain at each stage's barrier: 3-20% faster on the
//     256 x 96, 256 x 128 and 128 x 288 tiles), else two (256 x 192: a ring of three W stages beside two x stages,
//     W a stage further ahead, 3-6% faster); no registers are spent on staging. LDS rows are 128 B with the 16-byte chunks XOR-swizzled by (row / 2) mod
//     8, so the 16 rows that one ds_read_b128 touches land on 16 distinct bank groups. (Stages of 32 k with four
//     buffers were measured slower: twice the barriers, and no gain from the deeper DMA queue.) Half of a stage's
//     DMA instructions go out after the barrier that frees their buffer, the rest one per MFMA group of the next
//     stage: issued in one burst they fill the texture unit's command queue and stall the issuing waves.
//   * The operand with fewer fragments per wave stays in registers for a stage; the other one's fragments are read
//     two MFMA groups ahead, so LDS latency hides behind MFMAs.
//   * The body is compiled once per epilogue mode. The epilogue stages the accumulators through LDS a few fragment
//     columns at a time and applies the mode in a short rolled loop (the fully unrolled form was instruction-fetch
//     bound); its SiLU arithmetic is what remains of its cost.
//   * Persistent grid of one workgroup per CU. Tiles are first handed out in whole-tile waves of G (one tile per
//     workgroup, XCD-aware order so that the M tiles of one W tile run on the same XCD at the same time and share
//     its L2). The tiles left over (fewer than G) would leave most CUs idle for a whole tile time; instead their
//     K iterations are split evenly over Gs workgroups (stream-K). A workgroup whose range covers only part of a
//     tile writes its fp32 partial tile to a slot in the workspace; a second, small launch sums each split
//     tile's pieces in ascending K order (deterministic) and applies the epilogue. No workgroup ever waits for
//     another, and the GEMM carries no cross-workgroup code: an in-kernel last-arrival reduction was measured
//     (its registers cost the main loop spills, and its coherent stores bypassing L2 cost more than a launch).
#include "gemm_common.h"

namespace ojx {

namespace {

constexpr int kSkMaxPieces = 64;  // pieces one stream-K tile may be split into (host-enforced)


// Workgroup barrier for the DMA pipeline: LDS reads of this wave complete, then s_barrier. The DMAs of later
// stages stay in flight (a release fence on LDS would wait for every outstanding LDS DMA, vmcnt(0)); the caller
// has already waited, with an explicit vmcnt, for the DMAs of the stage this barrier publishes.
__device__ __forceinline__ void dma_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// First stream-K iteration of workgroup g when T iterations are shared by Gs workgroups (Gs <= T).
__device__ __forceinline__ int64_t sk_start(int64_t g, int64_t T, int64_t Gs) { return g * T / Gs; }
// The workgroup whose range holds iteration x: the largest g with sk_start(g) <= x.
__device__ __forceinline__ int64_t sk_owner(int64_t x, int64_t T, int64_t Gs) { return ((x + 1) * Gs + T - 1) / T - 1; }

// Instruction order of the main loop before its barrier (see the stage loop in gemm_sk_kernel). Group g of a stage
// (2 NR groups of NS MFMAs each: k32 step g / NR, streaming fragment g % NR) is preceded by its LDS reads: the
// streaming fragment of group g + PD and the step-1 stationary fragments assigned to it (fragment q is read in
// group q NR / NS).
template <int NS, int NR>
constexpr int sk_s1_reads(int g) {
  int n = 0;
  for (int q = 0; q < NS; ++q) n += (q * NR) / NS == g ? 1 : 0;
  return n;
}
template <int G, int NGA, int NS, int NR, int DPG, int NDG>
__device__ __forceinline__ void sk_sched() {  // NGA = groups before the barrier; DPG DMAs after the MFMAs of
  if constexpr (G < NGA) {                    // each of the first NDG groups
    __builtin_amdgcn_sched_group_barrier(0x100, 1 + sk_s1_reads<NS, NR>(G), 0);
    __builtin_amdgcn_sched_group_barrier(0x008, NS, 0);
    if constexpr (G < NDG) __builtin_amdgcn_sched_group_barrier(0x020, DPG, 0);
    sk_sched<G + 1, NGA, NS, NR, DPG, NDG>();
  }
}

}  // namespace

namespace {
// The kernel body, specialised per epilogue mode (EPI) so that the epilogue is straight code for one mode.
template <int FN, int FM, int WN, int WM, int EPI, bool PK>
__device__ __forceinline__ void sk_body(const GemmParams& p) {
  constexpr int BN = WN * FN * 16, BM = WM * FM * 16;
  constexpr int BK = 64, ROWS = BN + BM;
  constexpr int NW = WN * WM;
  constexpr int RB = 128;                       // LDS bytes per row (64 k of bf16)
  constexpr int STAGE = ROWS * RB;              // LDS bytes per stage
  // LDS stage buffers: 3 where they fit, so that the DMAs run two stages ahead and a wave's queue never drains at
  // the end of a stage; else 2 (one stage ahead)
  constexpr int NBUF = sk_nbuf(BN, BM);
  // ASYM (two stage buffers only): W in a ring of 3 stages and x in a ring of 2; a DMA batch carries x of its stage
  // and W of the next one, x first, so that W runs a stage further ahead and the wait for a stage leaves the next
  // stage's W in flight
  constexpr bool ASYM = sk_asym(BN, BM);
  constexpr int WST = BN * RB, XST = BM * RB;
  static_assert(sk_lds(BN, BM) == (ASYM ? 3 * WST + 2 * XST : NBUF * STAGE), "LDS layout");
  constexpr int NBLK = ROWS / 8;                // 8-row blocks per stage: one DMA instruction each
  constexpr int GPW = (NBLK + NW - 1) / NW;     // DMA instructions per wave and stage
  constexpr int GW = BN / 8 / NW;               // of which W blocks
  static_assert((BN / 8) % NW == 0 && BM % 16 == 0, "W blocks must fill whole DMA rounds");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // [2][ROWS][128 B], swizzled chunks

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % WN, wm = wave / WN;
  const int lr = lane & 15, lg = lane >> 4;

  // kernel arguments used in the loops, as plain scalars
  const int K = p.K, M = p.M, N = p.N;
  const int tiles_m = p.tiles_m;
  const int64_t ldw = p.ldw, ldx = p.ldx;
  const uint16_t* const Wp = p.W;
  const int nbw = N >> 4;       // its 16-row blocks
  const uint16_t* const Xp = p.X;

  // XCD-aware logical id: the hardware sends workgroup b to XCD b mod 8; consecutive logical ids share an XCD.
  const int G = gridDim.x, b = blockIdx.x;
  const int q = G >> 3, r = G & 7, xcd = b & 7;
  const int L = xcd * q + min(xcd, r) + (b >> 3);
  const int ipt = (K + BK - 1) / BK;  // K iterations (stages) per tile
  const int tiles = p.tiles_n * tiles_m;
  const int dp = p.dp_tiles;

  // DMA pattern: block gi = wave + i NW holds rows 8 gi .. 8 gi + 7; lane l fills row 8 gi + l / 8, physical
  // chunk l % 8, which holds logical chunk (l % 8) ^ ((row / 2) % 8). (row / 2) % 8 = 4 (gi % 2) + l / 16, and
  // gi % 2 = wave % 2 for every i (NW is even). Waves with fewer than GPW blocks repeat the last block (identical
  // bytes to the same place), so every wave issues GPW DMAs per stage.
  const int kcol = ((lane & 7) ^ ((((wave & 1) << 2) | (lane >> 4)) & 7)) * 8;  // k of this lane's chunk
  const int kcoll = ((lane & 7) ^ (((((NBLK - 1) & 1) << 2) | (lane >> 4)) & 7)) * 8;  // same, in the last block
  const uint32_t dW0 = (uint32_t)(((wave * 8 + (lane >> 3)) * ldw + kcol) * 2);
  const uint32_t dX0 = (uint32_t)(((wave * 8 + (lane >> 3)) * ldx + kcol) * 2);
  const uint32_t dXl = (uint32_t)((((NBLK - 1) * 8 - BN + (lane >> 3)) * ldx + kcoll) * 2);
  uint32_t stepW = (uint32_t)(NW * 8 * ldw * 2), stepX = (uint32_t)(NW * 8 * ldx * 2);
  // fragment reads: row r0 + lr (r0 a multiple of 16), logical chunk 4 s + lg of k32 step s
  const uint32_t ro0 = (uint32_t)(lr * RB + ((lg ^ (lr >> 1)) * 16));
  const uint32_t ro1 = (uint32_t)(lr * RB + (((4 + lg) ^ (lr >> 1)) * 16));
  const uint32_t wbase = (uint32_t)(wn * FN * 16 * RB), xbase = (uint32_t)(wm * FM * 16 * RB);
  // W and x of stage s in LDS (two or three stage buffers of W rows then x rows; ASYM: a W ring of 3, then an x
  // ring of 2)
  auto wptr = [&](int s) -> uint8_t* {
    if constexpr (ASYM) return smem + ((s + 3) % 3) * WST;  // s >= -1
    else return smem + (NBUF == 3 ? s % 3 : s & 1) * STAGE;
  };
  auto xptr = [&](int s) -> uint8_t* {
    if constexpr (ASYM) return smem + 3 * WST + (s & 1) * XST;
    else return smem + (NBUF == 3 ? s % 3 : s & 1) * STAGE + WST;
  };

  // stream-K range of this workgroup
  const int64_t T = (int64_t)(tiles - dp) * ipt;
  const int64_t Gs = p.sk_grid;
  const bool in_sk = T > 0 && L < Gs;
  const int64_t my0 = in_sk ? sk_start(L, T, Gs) : 0, my1 = in_sk ? sk_start(L + 1, T, Gs) : 0;

  f32x4 acc[FN][FM];
  int tau_dp = L;
  int64_t it = my0;
  while (true) {
    // ------------------------------------------------------------------ next segment: (tau, i0, i1)
    int tau, i0, i1, ts = -1;
    if (tau_dp < dp) {
      tau = tau_dp;
      i0 = 0;
      i1 = ipt;
      tau_dp += G;
    } else if (it < my1) {
      ts = (int)(it / ipt);
      i0 = (int)(it - (int64_t)ts * ipt);
      i1 = (int)min((int64_t)ipt, i0 + (my1 - it));
      it += i1 - i0;
      tau = dp + ts;
    } else {
      break;
    }
    tau = __builtin_amdgcn_readfirstlane(tau);
    i0 = __builtin_amdgcn_readfirstlane(i0);
    i1 = __builtin_amdgcn_readfirstlane(i1);
    const int n0 = (tau / tiles_m) * BN, m0 = (tau % tiles_m) * BM;
    const int kb = i0 * BK, ke = min(K, i1 * BK);
    const int nk = i1 - i0;
    // descriptors cover this tile's rows only: rows past N (or M) read zeros. A packed W (stage-major
    // [K/64][N/16][16][64], see ojx_pack_weight) is addressed through one descriptor over the whole buffer: W block
    // blk of a stage is 1 KiB at row block n0/16 + blk/2, half blk & 1, and blocks past N are skipped.
    const __amdgpu_buffer_rsrc_t rsW = PK ? make_rsrc(Wp, (int64_t)N * K * 2)
                                           : make_rsrc(Wp + (int64_t)n0 * ldw, (int64_t)min(BN, N - n0) * ldw * 2);
    const __amdgpu_buffer_rsrc_t rsX = make_rsrc(Xp + (int64_t)m0 * ldx, (int64_t)min(BM, M - m0) * ldx * 2);
    const __amdgpu_buffer_rsrc_t rsNone = make_rsrc(Wp, 0);
    const uint32_t dWp0 = (uint32_t)((((n0 >> 4) + (wave >> 1)) * 16 + (wave & 1) * 8 + (lane >> 3)) * 128 + kcol * 2);

#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // ------------------------------------------------------------------ main loop
    // DMAs lo .. hi-1 of the stage at k0 into buffer buf. The k offset (and, packed, the stage and block offset) is
    // wave-uniform and goes in the DMA's soffset; only the row-major block offset costs a vector add. A stage past
    // the segment reads zeros through an empty descriptor, W blocks past N (packed) likewise; only a partial last
    // stage (a K range that is not a multiple of 64) needs per-lane checks, on a separate path.
#define OJX_SK_DMA(s, lo, hi) OJX_SK_DMAW(s, lo, hi, false)
  // issue position j -> slot i: W slots (i < GW) first, or with ASYM the x slots first
#define OJX_SK_SLOT(j) (ASYM ? ((j) < GPW - GW ? GW + (j) : (j) - (GPW - GW)) : (j))
  // batch s: x of stage s and W of stage s (ASYM: s + 1); wonly: the W slots only
#define OJX_SK_DMAW(s, lo, hi, wonly)                                                                      \
  do {                                                                                                     \
    const int sx_ = (s), sw_ = ASYM ? sx_ + 1 : sx_;                                                       \
    const int kx_ = kb + sx_ * BK, kw_ = kb + sw_ * BK;                                                    \
    const bool livex_ = kx_ < ke, livew_ = kw_ < ke;                                                       \
    const bool partx_ = livex_ && kx_ + BK > ke, partw_ = livew_ && kw_ + BK > ke;                         \
    const uint32_t skx_ = (uint32_t)kx_ * 2u, skw_ = (uint32_t)kw_ * 2u;                                   \
    const uint32_t skp_ = (uint32_t)(kw_ >> 6) * (uint32_t)nbw * 2048u;                                    \
    const __amdgpu_buffer_rsrc_t rX_ = livex_ ? rsX : rsNone, rW_ = livew_ ? rsW : rsNone;                 \
    uint8_t* const wd_ = wptr(sw_);                                                                        \
    uint8_t* const xd_ = xptr(sx_) - BN * RB;  /* x block gi >= BN / 8 at xd_ + gi KiB */                   \
    /* keep the per-block offsets as one multiply-add each instead of GPW registers held across the loop */ \
    asm volatile("" : "+s"(stepW), "+s"(stepX));                                                           \
    _Pragma("unroll") for (int j = (lo); j < (hi); ++j) {                                                  \
      const int i = OJX_SK_SLOT(j);                                                                        \
      const bool real_ = GPW * NW == NBLK || wave + i * NW < NBLK;                                         \
      const int blk_ = real_ ? wave + i * NW : NBLK - 1;                                                   \
      if (i < GW) {                                                                                        \
        uint32_t o_ = PK ? dWp0 : dW0 + i * stepW;                                                         \
        if (PK && n0 + BN > N && n0 + blk_ * 8 >= N) o_ = kOOB;                                            \
        if (partw_ && kw_ + kcol >= ke) o_ = kOOB;                                                         \
        dma16s_nt(rW_, wd_ + blk_ * 1024, o_, PK ? skp_ + (uint32_t)(i * (NW / 2 * 2048)) : skw_);          \
      } else if (!(wonly)) {                                                                               \
        uint32_t o_ = real_ ? dX0 + (i - GW) * stepX : dXl;                                                \
        if (partx_ && kx_ + (real_ ? kcol : kcoll) >= ke) o_ = kOOB;                                       \
        dma16s(rX_, xd_ + blk_ * 1024, o_, skx_);                                                          \
      }                                                                                                    \
    }                                                                                                      \
  } while (0)
    // Fragment reads. The stationary operand is held for a whole k32 step (both steps' fragments in registers);
    // the streaming operand's fragments are read PD groups ahead of their MFMAs. The operand with fewer fragments
    // per wave is the stationary one: a stage then splits into more, smaller MFMA groups (2 NR groups of NS), which
    // gives the spread DMA issue more places to go. Holding the larger operand instead was measured 2-6% slower on
    // the 256x256, 256x192, 128x288 and 192x288 tiles, and makes the 256x288 tile spill.
    constexpr bool XST = FM < FN;
    constexpr int NS = XST ? FM : FN, NR = XST ? FN : FM;
#define OJX_SK_FRAG(sb, base, st, f) (*reinterpret_cast<const bf16x8*>((sb) + (base) + ((st) ? ro1 : ro0) + (f) * 16 * RB))
  // fragments of stage s: the stationary operand's (S) and the streaming operand's (R)
#define OJX_SK_S(s, st, q) OJX_SK_FRAG(XST ? xptr(s) : wptr(s), XST ? xbase : wbase, st, q)
#define OJX_SK_R(s, g) OJX_SK_FRAG(XST ? wptr(s) : xptr(s), XST ? wbase : xbase, (g) / NR, (g) % NR)
#define OJX_SK_MFMA(q, r, sv, rv)                                                                          \
  do {                                                                                                     \
    if constexpr (XST) acc[r][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rv, sv, acc[r][q], 0, 0, 0);    \
    else acc[q][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sv, rv, acc[q][r], 0, 0, 0);                  \
  } while (0)

    // Software pipeline across stages. A stage (64 k) is 2 NR groups (k32 step g / NR, streaming fragment g % NR)
    // of NS MFMAs. Stage t+1 is in flight by DMA while stage t is multiplied. The step-0 stationary fragments and
    // the first PD streaming fragments of stage t+1 are read right after the barrier that publishes it, while the
    // last PD groups of stage t (operands already in registers) keep the MFMA pipe busy; the buffer of stage t is
    // refilled with stage t+2 right after that barrier, by which point every wave has read it.
    constexpr int NGR = 2 * NR;
    constexpr int PD = NR < 2 ? NR : 2;  // prefetch distance in groups = trailing groups after the barrier
    constexpr int XR = PD + 1;           // streaming fragment ring
    // DMA issue: H0 of a stage's GPW DMA instructions right after the barrier that frees its buffer, the rest one
    // at a time after the MFMAs of the next stage's first groups. Issued all at once, the DMAs of 8 waves fill the
    // texture unit's command queue (measured full for a quarter of the kernel's cycles) and the waves stall at the
    // issue with the MFMA pipe idle. A DMA issued inside a stage must still land before that stage's barrier, so
    // spreading is limited to the groups that leave at least 16 MFMAs per SIMD (about 0.25 us) after the last one;
    // tiles with less room issue everything after the barrier.
    constexpr int NMG = NGR - PD;                  // groups before the barrier
    constexpr int NA = NMG - (16 + NS - 1) / NS;   // groups that may carry a DMA
    constexpr int H0 = NA <= 0 ? GPW : (GPW - NA > (GPW + 1) / 2 ? GPW - NA : (GPW + 1) / 2);
    constexpr int DPG = H0 < GPW ? 1 : 0;          // DMAs per group
    constexpr int NDG = GPW - H0;                  // groups that carry one
    if constexpr (ASYM) {
      OJX_SK_DMAW(-1, 0, GPW, true);  // W of stage 0
      OJX_SK_DMA(0, 0, GPW);          // x of stage 0, then W of stage 1
      OJX_SK_DMA(1, 0, H0);           // the rest of batch 1 in stage 0's groups (zeros past ke)
      wait_vmcnt<GW + H0>();          // W and x of stage 0 have landed
    } else if constexpr (NBUF == 3) {
      OJX_SK_DMA(0, 0, GPW);
      OJX_SK_DMA(1, 0, GPW);
      OJX_SK_DMA(2, 0, H0);           // the rest of stage 2 in stage 0's groups (zeros past ke)
      wait_vmcnt<GPW + H0>();         // stage 0 has landed; stages 1 and 2 may be in flight
    } else {
      OJX_SK_DMA(0, 0, GPW);
      OJX_SK_DMA(1, 0, H0);           // the rest of stage 1 in stage 0's groups (zeros past ke)
      wait_vmcnt<H0>();               // stage 0 has landed; stage 1 may be in flight
    }
    dma_barrier();
    bf16x8 s0c[NS], rn[PD];
#pragma unroll
    for (int q = 0; q < NS; ++q) s0c[q] = OJX_SK_S(0, 0, q);
#pragma unroll
    for (int d = 0; d < PD; ++d) rn[d] = OJX_SK_R(0, d);
    for (int t = 0; t < nk; ++t) {
      // the batch this stage's groups carry (t+1, or t+2 with three buffers), into buffers not read in this
      // stage; past the segment's last stage the DMAs read zeros into unused buffers
      const int ta = t + NBUF - 1;
      bf16x8 s1c[NS], rr[XR];
#pragma unroll
      for (int d = 0; d < PD; ++d) rr[d] = rn[d];
#pragma unroll
      for (int g = 0; g < NMG; ++g) {
#pragma unroll
        for (int qq = 0; qq < NS; ++qq)
          if ((qq * NR) / NS == g) s1c[qq] = OJX_SK_S(t, 1, qq);
        rr[(g + PD) % XR] = OJX_SK_R(t, g + PD);
#pragma unroll
        for (int qq = 0; qq < NS; ++qq) OJX_SK_MFMA(qq, g % NR, g < NR ? s0c[qq] : s1c[qq], rr[g % XR]);
        if constexpr (DPG > 0)
          if (g < NDG) OJX_SK_DMA(ta, H0 + g * DPG, min(GPW, H0 + (g + 1) * DPG));
      }
      sk_sched<0, NMG, NS, NR, DPG, NDG>();
      if (t + 1 < nk) {
        // this wave's DMAs of stage t+1 have landed (three buffers: those of stage t+2, all issued, may not have;
        // ASYM: the W of stage t+2 that batch t+1 issued last may not have)
        wait_vmcnt<NBUF == 3 ? GPW : ASYM ? GW : 0>();
        dma_barrier();    // every wave's has, and every wave's reads of stage t are done
        if constexpr (NBUF == 3) OJX_SK_DMA(t + 3, 0, H0);  // unconditional: the count above relies on it
        else if (t + 2 < nk) OJX_SK_DMA(t + 2, 0, H0);
#pragma unroll
        for (int qq = 0; qq < NS; ++qq) s0c[qq] = OJX_SK_S(t + 1, 0, qq);
#pragma unroll
        for (int d = 0; d < PD; ++d) rn[d] = OJX_SK_R(t + 1, d);
      }
#pragma unroll
      for (int g = NGR - PD; g < NGR; ++g)
#pragma unroll
        for (int qq = 0; qq < NS; ++qq) OJX_SK_MFMA(qq, g % NR, s1c[qq], rr[g % XR]);
    }
    wait_vmcnt<0>();  // the last stage's zero-fill DMAs, before LDS is reused
    dma_barrier();  // the next segment's first DMAs reuse buffer 0
#undef OJX_SK_FRAG
#undef OJX_SK_S
#undef OJX_SK_R
#undef OJX_SK_MFMA
#undef OJX_SK_DMA
#undef OJX_SK_DMAW
#undef OJX_SK_SLOT

    // ------------------------------------------------------------------ partial tile: to its slot
    if (i0 != 0 || i1 != ipt) {
      // Pieces of stream-K tile ts belong to workgroups g0..g1 in K order; a workgroup keeps a tile's piece in
      // slot 2g if the tile is where its range starts, else (its range ends inside the tile) in slot 2g+1.
      // gemm_sk_fixup_kernel, launched right after this kernel, sums the pieces and applies the epilogue.
      // A slot holds the tile row-major ([BM][BN] fp32), so that the row pass of the residual epilogue reads each
      // row's columns contiguously.
      const int64_t x0 = (int64_t)ts * ipt;
      float* slot = p.sk_ws + (2 * L + (my0 >= x0 ? 0 : 1)) * (int64_t)(BN * BM) +
                    (int64_t)(wm * FM * 16 + lr) * BN + wn * FN * 16 + lg * 4;
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) *reinterpret_cast<f32x4*>(slot + j * 16 * BN + i * 16) = acc[i][j];
      continue;
    }

    // ------------------------------------------------------------------ epilogue
    // Through LDS, P fragment columns at a time: the waves stage acc[i..i+P-1][*] (BM rows x WN strips of 16 P
    // columns), then every thread applies the epilogue to IMAX items of 4 (SiLU: 8) consecutive columns, unrolled
    // so that the items' LDS reads, math and stores overlap. The pass loop stays rolled: fully unrolled over the
    // FN x FM fragments, the epilogue is tens of KB of straight-line code run once per tile, whose instruction
    // fetches were measured to cost up to a quarter of the tile time.
    {
      constexpr int LDSB = 2 * STAGE;
      constexpr int COLB = BM * (WN * 16 + 4) * 4;
      constexpr int P = (FN % 4 == 0 && 4 * COLB <= LDSB) ? 4 : (FN % 2 == 0 && 2 * COLB <= LDSB) ? 2 : 1;
      static_assert(COLB <= LDSB, "one staged fragment column must fit the LDS");
      constexpr int SROW = WN * 16 * P + 4;  // floats per staged row (padded against bank conflicts)
      constexpr bool SILU = EPI == EPI_SILU;
      constexpr int CW = SILU ? 8 : 4;       // columns per item
      constexpr int ITEMS = BM * WN * 16 * P / CW;
      constexpr int IMAX = (ITEMS + 64 * NW - 1) / (64 * NW);
      float* const stg = reinterpret_cast<float*>(smem);
#pragma nounroll
      for (int i = 0; i < FN; i += P) {
#pragma unroll
        for (int ii = 0; ii < FN; ii += P)
          if (ii == i) {
#pragma unroll
            for (int pp = 0; pp < P; ++pp)
#pragma unroll
              for (int j = 0; j < FM; ++j)
                *reinterpret_cast<f32x4*>(stg + ((wm * FM + j) * 16 + lr) * SROW + (wn * P + pp) * 16 + lg * 4) =
                    acc[ii + pp][j];
          }
        dma_barrier();
        constexpr int IB = IMAX < 4 ? IMAX : 4;  // items in flight per thread (registers beside acc)
#pragma unroll
        for (int k0 = 0; k0 < IMAX; k0 += IB) {
          f32x4 v[IB], u[IB];
#pragma unroll
          for (int k = 0; k < IB; ++k) {
            const int e = min(tid + (k0 + k) * 64 * NW, ITEMS - 1);
            const float* src = stg + (e / (WN * P * 16 / CW)) * SROW + (e % (WN * P * 16 / CW)) * CW;
            v[k] = *reinterpret_cast<const f32x4*>(src);
            if constexpr (SILU) u[k] = *reinterpret_cast<const f32x4*>(src + 4);
            else u[k] = v[k];
          }
#pragma unroll
          for (int k = 0; k < IB; ++k) {
            const int e = tid + (k0 + k) * 64 * NW;
            if (k0 + k >= IMAX || (ITEMS % (64 * NW) != 0 && e >= ITEMS)) continue;
            const int m = e / (WN * P * 16 / CW), cc = (e % (WN * P * 16 / CW)) * CW;  // staged column
            const int sp = cc >> 4;                                                   // strip = wn * P + pp
            const int n = n0 + ((sp / P) * FN + i + sp % P) * 16 + (cc & 15);
            store4(p, EPI, 0, m0 + m, n, true, v[k], u[k]);
          }
        }
        dma_barrier();
      }
    }
  }
}

}  // namespace

template <int FN, int FM, int WN, int WM>
__global__ void __launch_bounds__(64 * WN * WM) gemm_sk_kernel(const GemmParams p, const int epi) {
  if (p.wpk) {  // W in the packed layout
    if (epi == EPI_SILU) sk_body<FN, FM, WN, WM, EPI_SILU, true>(p);
    else if (epi == EPI_RESID) sk_body<FN, FM, WN, WM, EPI_RESID, true>(p);
    else sk_body<FN, FM, WN, WM, EPI_BF16, true>(p);  // the host routes EPI_F32 (split-K planes) to other families
  } else {
    if (epi == EPI_SILU) sk_body<FN, FM, WN, WM, EPI_SILU, false>(p);
    else if (epi == EPI_RESID) sk_body<FN, FM, WN, WM, EPI_RESID, false>(p);
    else sk_body<FN, FM, WN, WM, EPI_BF16, false>(p);
  }
}

// Second pass of a stream-K plan: a tile that was split sums its pieces in K order, ((p0 + p1) + p2) + ..., and
// applies the epilogue; a tile done whole by one workgroup was finished by the GEMM. One workgroup of 256 threads per
// split tile and block of 16 rows (one per tile left this pass bound by the bandwidth of a few dozen CUs); each
// thread takes 8 consecutive columns of a row (the slots are row-major), so its loads are 32 contiguous bytes and a
// packed gate/up group of 8 columns is whole in one thread. The pieces are visible here because the GEMM launch has
// ended.
template <int FN, int FM, int WN, int WM>
__global__ void __launch_bounds__(256) gemm_sk_fixup_kernel(const GemmParams p, const int epi) {
  constexpr int BN = WN * FN * 16, BM = WM * FM * 16, BK = 64, RB = BM / 16;
  constexpr int ITEMS = 16 * BN / 8;
  __shared__ int s_slot[kSkMaxPieces];
  const int tid = threadIdx.x;
  const int ipt = (p.K + BK - 1) / BK;
  const int ts = blockIdx.x / RB, rb = blockIdx.x % RB;
  const int64_t T = (int64_t)(p.tiles_n * p.tiles_m - p.dp_tiles) * ipt;
  const int64_t Gs = p.sk_grid;
  const int64_t x0 = (int64_t)ts * ipt;
  const int64_t g0 = sk_owner(x0, T, Gs), g1 = sk_owner(x0 + ipt - 1, T, Gs);
  if (g0 == g1) return;
  const int np = (int)(g1 - g0 + 1);  // at most kSkMaxPieces (the host sizes the grid so)
  if (tid < np) {
    const int64_t g = g0 + tid;
    s_slot[tid] = (int)(2 * g + (sk_start(g, T, Gs) >= x0 ? 0 : 1));
  }
  __syncthreads();
  const int tau = p.dp_tiles + ts;
  const int n0 = (tau / p.tiles_m) * BN, m0 = (tau % p.tiles_m) * BM;
  for (int it = tid; it < ITEMS; it += 256) {
    const int r = rb * 16 + it / (BN / 8), c = (it % (BN / 8)) * 8;
    const float* src = p.sk_ws + (int64_t)r * BN + c;
    f32x4 a = *reinterpret_cast<const f32x4*>(src + (int64_t)s_slot[0] * (BN * BM));
    f32x4 b = *reinterpret_cast<const f32x4*>(src + (int64_t)s_slot[0] * (BN * BM) + 4);
    for (int k = 1; k < np; ++k) {
      const f32x4 ca = *reinterpret_cast<const f32x4*>(src + (int64_t)s_slot[k] * (BN * BM));
      const f32x4 cb = *reinterpret_cast<const f32x4*>(src + (int64_t)s_slot[k] * (BN * BM) + 4);
      a += ca;
      b += cb;
    }
    const int m = m0 + r, n = n0 + c;
    if (epi == EPI_SILU) {
      store4(p, EPI_SILU, 0, m, n, true, a, b);  // columns n .. n+3 gate, n+4 .. n+7 up
    } else {
      store4(p, epi, 0, m, n, true, a, a);
      store4(p, epi, 0, m, n + 4, true, b, b);
    }
  }
}

// Second pass of a stream-K plan with the residual epilogue, fused with the RMSNorm of the rows: one workgroup per
// output row m, N/8 threads, 8 consecutive columns each. For a column of a split tile the thread sums the tile's
// pieces in K order exactly as gemm_sk_fixup_kernel does and writes h = bf16(residual + bf16(sum)); columns of
// tiles done whole were written by the GEMM and are read back. Then hn = RMSNorm(h) * w1 with the arithmetic of
// add_rmsnorm_k, so the result is bit-identical to GEMM -> fixup -> add_rmsnorm in one launch fewer, with h not
// read back for the split tiles (the reference: bmm, then add_rmsnorm_sk2, src/fastmodel.py:196-203).
template <int FN, int FM, int WN, int WM>
__global__ void __launch_bounds__(1024) gemm_sk_fixup_rmsnorm_kernel(const GemmParams p, const float* w1,
                                                                    const int32_t* rowmask, float eps,
                                                                    uint16_t* hn_out) {
  constexpr int BN = WN * FN * 16, BM = WM * FM * 16, BK = 64;
  __shared__ float red[16];
  const int m = blockIdx.x, n8 = threadIdx.x * 8;
  const int N = p.N;
  const int ipt = (p.K + BK - 1) / BK;
  const int64_t T = (int64_t)(p.tiles_n * p.tiles_m - p.dp_tiles) * ipt;
  const int64_t Gs = p.sk_grid;
  const int tn = n8 / BN, c = n8 % BN;
  const int tm = m / BM, mm = m % BM;
  const int tau = tn * p.tiles_m + tm;
  uint16_t* const h = static_cast<uint16_t*>(p.out) + (int64_t)m * p.ldo + n8;
  float v[8];
  bool split = false;
  int64_t g0 = 0, g1 = 0, x0 = 0;
  if (tau >= p.dp_tiles && T > 0) {
    x0 = (int64_t)(tau - p.dp_tiles) * ipt;
    g0 = sk_owner(x0, T, Gs);
    g1 = sk_owner(x0 + ipt - 1, T, Gs);
    split = g0 != g1;
  }
  if (split) {
    const float* base = p.sk_ws + (int64_t)mm * BN + c;  // row-major slots: columns c .. c+7 of tile row mm
    auto slot = [&](int64_t g) { return (int64_t)(2 * g + (sk_start(g, T, Gs) >= x0 ? 0 : 1)) * (BN * BM); };
    f32x4 a = *reinterpret_cast<const f32x4*>(base + slot(g0));
    f32x4 b = *reinterpret_cast<const f32x4*>(base + slot(g0) + 4);
    for (int64_t g = g0 + 1; g <= g1; ++g) {
      const f32x4 ca = *reinterpret_cast<const f32x4*>(base + slot(g));
      const f32x4 cb = *reinterpret_cast<const f32x4*>(base + slot(g) + 4);
      a += ca;
      b += cb;
    }
    const uint4 ra = *reinterpret_cast<const uint4*>(p.res + (int64_t)m * p.ldr + n8);
    const uint32_t rw[4] = {ra.x, ra.y, ra.z, ra.w};
    const float s[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = rbf(bf2f(rw[e] & 0xffffu) + rbf(s[2 * e]));
      v[2 * e + 1] = rbf(bf2f(rw[e] >> 16) + rbf(s[2 * e + 1]));
    }
    *reinterpret_cast<uint4*>(h) = make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]),
                                              pack2(v[6], v[7]));
  } else {
    const uint4 ha = *reinterpret_cast<const uint4*>(h);
    const uint32_t hw[4] = {ha.x, ha.y, ha.z, ha.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[2 * e] = bf2f(hw[e] & 0xffffu); v[2 * e + 1] = bf2f(hw[e] >> 16); }
  }
  (void)N;
  const float4 wa = *reinterpret_cast<const float4*>(w1 + n8), wb = *reinterpret_cast<const float4*>(w1 + n8 + 4);
  rmsnorm_row8(v, wa, wb, rowmask == nullptr || rowmask[m] != 0, eps, p.N, red, hn_out + (int64_t)m * p.N + n8);
}

}  // namespace ojx

namespace ojx {
// Tile shapes of this family (registered in gemm.hip's tile table): BN x BM = (WN*FN*16) x (WM*FM*16).
template __global__ void gemm_sk_kernel<8, 4, 2, 4>(const GemmParams, const int);  // 256 x 256
template __global__ void gemm_sk_fixup_kernel<8, 4, 2, 4>(const GemmParams, const int);
template __global__ void gemm_sk_fixup_rmsnorm_kernel<8, 4, 2, 4>(const GemmParams, const float*, const int32_t*,
                                                                  float, uint16_t*);
template __global__ void gemm_sk_kernel<4, 9, 4, 2>(const GemmParams, const int);  // 256 x 288
template __global__ void gemm_sk_fixup_kernel<4, 9, 4, 2>(const GemmParams, const int);
template __global__ void gemm_sk_fixup_rmsnorm_kernel<4, 9, 4, 2>(const GemmParams, const float*, const int32_t*,
                                                                  float, uint16_t*);
template __global__ void gemm_sk_kernel<4, 4, 4, 2>(const GemmParams, const int);  // 256 x 128
template __global__ void gemm_sk_fixup_kernel<4, 4, 4, 2>(const GemmParams, const int);
template __global__ void gemm_sk_fixup_rmsnorm_kernel<4, 4, 4, 2>(const GemmParams, const float*, const int32_t*,
                                                                  float, uint16_t*);
template __global__ void gemm_sk_kernel<4, 6, 4, 2>(const GemmParams, const int);  // 256 x 192
template __global__ void gemm_sk_fixup_kernel<4, 6, 4, 2>(const GemmParams, const int);
template __global__ void gemm_sk_fixup_rmsnorm_kernel<4, 6, 4, 2>(const GemmParams, const float*, const int32_t*,
                                                                  float, uint16_t*);
template __global__ void gemm_sk_kernel<4, 3, 4, 2>(const GemmParams, const int);  // 256 x 96
template __global__ void gemm_sk_fixup_kernel<4, 3, 4, 2>(const GemmParams, const int);
template __global__ void gemm_sk_fixup_rmsnorm_kernel<4, 3, 4, 2>(const GemmParams, const float*, const int32_t*,
                                                                  float, uint16_t*);
template __global__ void gemm_sk_kernel<2, 9, 4, 2>(const GemmParams, const int);  // 128 x 288
template __global__ void gemm_sk_fixup_kernel<2, 9, 4, 2>(const GemmParams, const int);
template __global__ void gemm_sk_fixup_rmsnorm_kernel<2, 9, 4, 2>(const GemmParams, const float*, const int32_t*,
                                                                  float, uint16_t*);
template __global__ void gemm_sk_kernel<3, 9, 4, 2>(const GemmParams, const int);  // 192 x 288
template __global__ void gemm_sk_fixup_kernel<3, 9, 4, 2>(const GemmParams, const int);
template __global__ void gemm_sk_fixup_rmsnorm_kernel<3, 9, 4, 2>(const GemmParams, const float*, const int32_t*,
                                                                  float, uint16_t*);
}  // namespace ojx
