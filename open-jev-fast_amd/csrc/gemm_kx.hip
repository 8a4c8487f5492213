// bf16 projection GEMM for gfx950 with K-interleaved wave pairs: y[M,N] = x[M,K] . W[N,K]^T, fp32 accumulation on
// v_mfma_f32_16x16x32_bf16, epilogues fused into the store (same modes as gemm.hip).
//
// Replaces the reference's cuBLASLt GEMM (src/lt.cpp:43-55, through _mm, src/fastmodel.py:168-175) at the M where
// a projection needs whole-M tiles: the tile covers all of x (M <= BM), so each W row is read from HBM once, and
// BN is chosen so that the tile count fills the 256 CUs (144 W rows for the 34816-row gate-up: 242 tiles).
//
// Why this shape of kernel:
//   * The 16x16 fragments of a BN x BM tile do not split evenly over 8 waves for the tile sizes that fill the chip
//     (9 x 18 fragments for 144 x 288). Instead the tile is split over the four SIMDs (group g = wave & 3): group g
//     owns W fragments 0..FW-1 times x fragments g*FX .. g*FX+FX-1, plus an equal share of the XE x fragments left
//     over (x fragment 4*FX + ..., EW of its W fragments). The two waves of a group (wave g and wave g+4) own the
//     same fragments and interleave K: within every 64-k stage, wave g multiplies the first 32 k and wave g+4 the
//     second. Every wave therefore carries FW*FX + EW accumulators (41 for 144 x 288, 164 registers) and reads
//     FW + FX + 1 fragments per k32 step: 14 LDS fragment reads per 41 MFMAs, against 24 per 54 for eight 48 x 144
//     wave tiles, with two waves per SIMD to hide LDS latency and barriers.
//   * The pair's partial sums are added through LDS at the end of the tile (two exchanges of half the fragments),
//     so each wave then stores half of its group's outputs. The sum over k is (even 32-k blocks) + (odd 32-k
//     blocks): deterministic, but a different rounding order from the other tile families.
//   * Operands reach LDS by DMA (buffer_load ... lds, 16 B per lane, one 8-row x 128 B block per wave instruction)
//     in stages of 64 k: an x ring of XD stages and a W ring of XD + 1, the DMAs XD stages ahead of the stage being
//     multiplied (XD = 2 on most tiles; 4 on a 128 x 64 tile for the weight stream at M = 64). LDS rows are 128 B
//     with the 16-byte chunks XOR-swizzled by (row / 2) mod 8, so the 16 rows one ds_read_b128 touches hit distinct
//     banks.
//     Half of a stage's DMA instructions go out right after the barrier that frees their buffer, the rest one per
//     MFMA group of the following groups.
//   * A wave walks its W fragments starting at its first extra fragment (rotated order), so the extra MFMAs sit
//     in the first EW groups of every stage for every wave: straight-line code for all groups.
#include "gemm_common.h"

namespace ojx {

namespace {

__device__ __forceinline__ void kx_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int FW, int FX, int XE, int XD>
struct KxShape {
  static constexpr int BN = 16 * FW, BM = 16 * (4 * FX + XE);
  // x ring depth XD = the prefetch distance in stages of 64 k; the W ring has one stage more (a W slot is free as
  // soon as its stage's W fragments are read, an x slot only once every wave holds its x fragments in registers)
  static constexpr int RB = 128, WD = XD + 1;
  static constexpr int LDS = (WD * BN + XD * BM) * RB;            // W ring + x ring
  static constexpr int NW = 8;
  static constexpr int EW = XE == 0 ? 0 : XE == 1 ? (FW + 3) / 4 : (FW + 1) / 2;  // extra W fragments per group
  static constexpr int NX = FX + (XE > 0 ? 1 : 0);                                  // x fragments per wave
  static constexpr int NACC = FW * FX + EW;                                         // accumulators per wave
  static constexpr int HF = (NACC + 1) / 2;                                         // fragments reduced by wave g
  static_assert(XE >= 0 && XE <= 2, "0..2 leftover x fragments");
  static_assert(XD >= 2, "x ring of two stages or more");
  static_assert(4 * HF * 64 * 16 <= LDS, "the pair exchange must fit the stage buffers");
  static_assert(LDS <= 160 * 1024, "LDS");
};

// Full-attention prep epilogue of the QKV in-projection (EPI_FATTN; 256-row tiles = one head block, FX x fragments
// per SIMD group, no leftover fragments). After the pair reduction wave g (h = 0) holds dims 0..127 and wave g+4
// (h = 1) dims 128..255 of the group's 16 FX rows. The 256-row block n0 / 256 is a q head (even blocks below
// 2 HQ), the gate of that head (odd blocks), a k head, or a v head. q and k: proj = bf16(acc), RMSNorm over the
// head's 256 dims (each wave sums its half over its lanes, the pair adds through LDS), weight qw1 / kw1, then the
// rotate-half RoPE on the first RD = 64 dims (the partner of dim d is in fragment d/16 +- 2 of the same lane),
// stored head-major; gate and v: proj stored as it is. Same arithmetic as fullattn_prep_k (prep.hip), the
// reference's fullattn_prep2_k (src/kernels.cu:302-355), except the order in which the sum of squares is added.
// H is the wave's half as a template argument: the accumulators are then indexed by constants and stay in registers
// (an index computed from the wave id would put the whole array on the stack).
template <int FW, int FX, int H>
__device__ __forceinline__ void kx_fattn_epilogue(const GemmParams& p, f32x4 (&acc)[FW][FX], int g, int lane,
                                                  int m0, int n0, uint8_t* smem) {
  static_assert(FW == 16, "one 256-dim head per tile");
  constexpr int h = H;
  constexpr int D = 256, RDF = 2;  // RoPE dims = 64 = 4 fragments; partner fragment distance 2
  const FattnParams& fa = p.fa;
  const int lr = lane & 15, lg = lane >> 4;
  const int cb = n0 / D;
  const int type = cb < 2 * fa.HQ ? (cb & 1) : (cb < 2 * fa.HQ + fa.HKV ? 2 : 3);  // 0 q, 1 gate, 2 k, 3 v
  const int hh = cb < 2 * fa.HQ ? cb >> 1 : (type == 2 ? cb - 2 * fa.HQ : cb - 2 * fa.HQ - fa.HKV);
  const int M = p.M;
  constexpr int p0 = h * 8;  // this wave's fragments (positions = W fragments) p0 .. p0+7
  if (type == 1 || type == 3) {
#pragma unroll
    for (int pp = 0; pp < 8; ++pp)
#pragma unroll
      for (int xi = 0; xi < FX; ++xi) {
        const int m = m0 + (g * FX + xi) * 16 + lr;
        if (m >= M) continue;
        const f32x4 v = acc[p0 + pp][xi];
        const uint2 o = make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
        const int d = (p0 + pp) * 16 + lg * 4;
        uint16_t* dst = type == 1 ? fa.gate + (int64_t)m * (fa.HQ * D) + hh * D + d
                                  : fa.vt + ((int64_t)hh * M + m) * D + d;
        *reinterpret_cast<uint2*>(dst) = o;
      }
    return;
  }
  // q or k: bf16 proj values, the head's sum of squares per row
  float ss[FX];
#pragma unroll
  for (int xi = 0; xi < FX; ++xi) {
    float s = 0.f;
#pragma unroll
    for (int pp = 0; pp < 8; ++pp)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = rbf(acc[p0 + pp][xi][e]);
        acc[p0 + pp][xi][e] = x;
        s += x * x;
      }
    s += __shfl_xor(s, 16);
    s += __shfl_xor(s, 32);
    ss[xi] = s;
  }
  float* red = reinterpret_cast<float*>(smem + 96 * 1024);  // past the pair exchange area
#pragma unroll
  for (int xi = 0; xi < FX; ++xi)
    if (lg == 0) red[((g * 2 + h) * FX + xi) * 16 + lr] = ss[xi];
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  const float* w1 = type == 0 ? fa.qw1 : fa.kw1;
  uint16_t* const out = type == 0 ? fa.qt : fa.kt;
#pragma unroll
  for (int xi = 0; xi < FX; ++xi) {
    const float tot = ss[xi] + red[((g * 2 + (h ^ 1)) * FX + xi) * 16 + lr];
    const float r = rsqrtf(tot / (float)D + fa.eps);
    const int m = m0 + (g * FX + xi) * 16 + lr;
    float nv[8][4];
#pragma unroll
    for (int pp = 0; pp < 8; ++pp) {
      const float4 wv = *reinterpret_cast<const float4*>(w1 + (p0 + pp) * 16 + lg * 4);
      const float wa[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) nv[pp][e] = rbf((acc[p0 + pp][xi][e] * r) * wa[e]);
    }
    if (m >= M) continue;
#pragma unroll
    for (int pp = 0; pp < 8; ++pp) {
      float o[4];
      const int d = (p0 + pp) * 16 + lg * 4;
      if (h == 0 && pp < 2 * RDF) {  // the rotate-half RoPE on dims 0..63
        const uint2 ca = *reinterpret_cast<const uint2*>(fa.cosb + (int64_t)m * fa.RD + d);
        const uint2 sa = *reinterpret_cast<const uint2*>(fa.sinb + (int64_t)m * fa.RD + d);
        const float c[4] = {bf2f(ca.x & 0xffffu), bf2f(ca.x >> 16), bf2f(ca.y & 0xffffu), bf2f(ca.y >> 16)};
        const float sn[4] = {bf2f(sa.x & 0xffffu), bf2f(sa.x >> 16), bf2f(sa.y & 0xffffu), bf2f(sa.y >> 16)};
        const int q = pp < RDF ? pp + RDF : pp - RDF;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float rh = pp < RDF ? -nv[q][e] : nv[q][e];
          o[e] = rbf(rbf(nv[pp][e] * c[e]) + rbf(rh * sn[e]));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = nv[pp][e];
      }
      *reinterpret_cast<uint2*>(out + ((int64_t)hh * M + m) * D + d) = make_uint2(pack2(o[0], o[1]), pack2(o[2], o[3]));
    }
  }
}

// REV (two leftover x fragments only): the group walks its W fragments from the last one down, so that its extra
// fragments (the upper half) come first; the other groups walk upwards. Either way the walk is static code.
template <int FW, int FX, int XE, int XD, int EPI, bool REV, bool PK>
__device__ __forceinline__ void kx_body(const GemmParams& p) {
  using S = KxShape<FW, FX, XE, XD>;
  constexpr int BN = S::BN, BM = S::BM, RB = S::RB, NW = S::NW;
  // DMA waves: the waves that issue the operand DMAs. Only the second wave of each SIMD (h = 1) issues them, so a
  // wave stalled at a full texture-unit queue leaves its SIMD partner free to keep the MFMA pipe busy (measured
  // 3-6% faster than DMAs from all 8 waves on the 144 x 64, 144 x 128 and 128 x 288 tiles).
  constexpr int DWV = 4;
  constexpr int GPW = ((BN + BM) / 8 + DWV - 1) / DWV;
  constexpr int EW = S::EW, NX = S::NX, NACC = S::NACC, HF = S::HF;
  constexpr int BK = 64;

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // W ring, then x double buffer

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = wave & 3, h = wave >> 2;
  const int lr = lane & 15, lg = lane >> 4;

  // XCD-aware logical tile id (workgroup b runs on XCD b mod 8); M tile fastest, then split, then N tile.
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

  // row-major W: this tile's rows only (rows past N read zeros); packed W: the whole buffer, blocks past N skipped
  const __amdgpu_buffer_rsrc_t rsW = PK ? make_rsrc(p.W, (int64_t)p.N * p.K * 2)
                                           : make_rsrc(p.W + (int64_t)n0 * p.ldw, (int64_t)min(BN, p.N - n0) * p.ldw * 2);
  const int nbw = p.N >> 4;  // 16-row blocks of the packed W
  const __amdgpu_buffer_rsrc_t rsX = make_rsrc(p.X + (int64_t)m0 * p.ldx, (int64_t)min(BM, p.M - m0) * p.ldx * 2);

  // ------------------------------------------------------------------ fragment ownership
  // extra fragments: x fragment xe, W fragments wstart .. wstart + EW - 1 (walked first)
  const int xe = 4 * FX + (XE == 2 ? (g >> 1) : 0);
  const int wnom = XE == 1 ? g * EW : XE == 2 ? (g & 1) * EW : 0;  // first extra this group stores
  const int wstart = XE == 2 ? (REV ? FW - EW : 0) : min(wnom, FW - EW);
  // W fragment at walk position pp
  auto wfrag = [&](int pp) -> int {
    if constexpr (XE == 2) return REV ? FW - 1 - pp : pp;
    const int j = wstart + pp;
    return j >= FW ? j - FW : j;
  };
  // LDS byte offsets (within a stage) of this lane's reads for its k half: row r0 + lr, chunk 4h + lg swizzled
  const uint32_t ro = (uint32_t)(lr * RB + (((4 * h + lg) ^ (lr >> 1)) & 7) * 16);
  uint32_t woff[FW];
#pragma unroll
  for (int pp = 0; pp < FW; ++pp) woff[pp] = (uint32_t)(wfrag(pp) * 16 * RB) + ro;
  uint32_t xoff[NX];
#pragma unroll
  for (int i = 0; i < FX; ++i) xoff[i] = (uint32_t)((g * FX + i) * 16 * RB) + ro;
  if constexpr (XE > 0) xoff[FX] = (uint32_t)(xe * 16 * RB) + ro;

  // ------------------------------------------------------------------ LDS rings and DMA pattern
  // LDS: a ring of WD = XD + 1 stages of W (BN rows x 128 B = 64 k) and a ring of XD stages of x (BM rows), 16-byte
  // chunks XOR-swizzled by (row / 2) mod 8 within each region. A wave reads its x fragments of a stage into
  // registers right after the barrier that publishes the stage and keeps them for the whole stage, so a second
  // barrier a few MFMA groups later frees that x buffer: the DMAs issued then (batch t, issued as stage t begins)
  // fetch x and W of stage t+XD. Both operands get XD stages to arrive; the weights come from HBM, x (the same rows
  // for every workgroup) mostly from L2, and a wave's DMAs complete in issue order, so the x and W traffic share one
  // queue.
  constexpr int WST = BN * RB, XST = BM * RB;
  uint8_t* const wring = smem;
  uint8_t* const xring = smem + S::WD * WST;
  constexpr int XB = BM / 8, WB = BN / 8, NB = XB + WB;
  // Batch slot i (i < GPW) of DMA wave dw fetches block c = dw + DWV i of a stage: x block c if c < XB, else W block
  // c - XB; past the last block a wave repeats that block (same bytes to the same place), so every DMA wave issues
  // GPW DMAs per batch. Only the stage changes from batch to batch: the stage's byte offset is a wave-uniform SGPR
  // passed as the DMA's soffset, and a stage past the end reads through an empty descriptor (zeros). All blocks of
  // a wave have the parity of dw (DWV and XB are even), hence the same 16-byte chunk swizzle, so a slot's lane
  // offset is linear in i: one VGPR for x (vx0), one for W (vwr, at the first slot that is W for every wave), a
  // scalar step each, and one VGPR for the repeated last block. Slots whose kind is the same for every wave are
  // told apart at compile time; at most one slot is x for some waves and W for others.
  const bool dmaw = wave >= NW - DWV;
  const int dw = dmaw ? wave - (NW - DWV) : 0;
  const int lrow = lane >> 3;
  auto swz = [&](int par) { return ((lane & 7) ^ ((par << 2) | (lane >> 4))) * 8; };  // k of the lane's chunk
  const int kc = swz(dw & 1), kcl = swz((WB - 1) & 1);
  auto wlane = [&](int blk, int k) -> uint32_t {  // lane offset of W block blk at stage 0 (chunk k)
    if constexpr (PK) return (uint32_t)(((((n0 >> 4) + (blk >> 1)) * 16 + (blk & 1) * 8 + lrow) * 64 + k) * 2);
    else return (uint32_t)(((int64_t)(blk * 8 + lrow) * p.ldw + kb + k) * 2);
  };
  constexpr int IW = (XB + DWV - 1) / DWV;  // first slot that is W for every wave
  const uint32_t vx0 = (uint32_t)(((int64_t)(dw * 8 + lrow) * p.ldx + kb + kc) * 2);
  const uint32_t vwr = wlane(dw + DWV * IW - XB, kc), vlast = wlane(WB - 1, kcl);
  const uint32_t sxs = (uint32_t)(DWV * 8 * p.ldx * 2);
  const uint32_t sws = PK ? (uint32_t)(DWV * 1024) : (uint32_t)(DWV * 8 * p.ldw * 2);
  const __amdgpu_buffer_rsrc_t rsNone = make_rsrc(p.W, 0);
  const bool ragged = ((ke - kb) & (BK - 1)) != 0;  // the last stage is partial: lanes past ke read zeros
  const bool wedge = PK && n0 + BN > p.N;            // packed: some W blocks of this tile are past N
  // DMAs lo .. hi-1 of the batch that fetches stage st (x into x slot st & 1, W into W slot st % WD)
  auto dma = [&](int st, int lo, int hi) {
    if (!dmaw) return;
    // the issuing wave goes first while it issues (its SIMD partner's MFMAs wait a few cycles, the DMAs leave
    // sooner): measured 2-5% faster on the 144 x 128 and 128 x 288 tiles
    __builtin_amdgcn_s_setprio(2);
    const bool ok = st < nk;
    const uint32_t sx = (uint32_t)(st * BK * 2);  // kb is in the lane offsets
    const uint32_t sw = PK ? (uint32_t)(((kb >> 6) + st) * nbw * 2048) : sx;
    const __amdgpu_buffer_rsrc_t rX = ok ? rsX : rsNone, rW = ok ? rsW : rsNone;
    uint8_t* const xd = xring + (st % XD) * XST;
    uint8_t* const wd = wring + (st % S::WD) * WST;
    const bool tail = ragged && st == nk - 1;  // rare
#pragma unroll
    for (int i = 0; i < GPW; ++i) {
      if (i < lo || i >= hi) continue;
      const bool allx = DWV * i + DWV - 1 < XB, allw = DWV * i >= XB;  // compile-time after unrolling
      const bool mayend = DWV * i + DWV > NB;                          // compile-time: slot may run past NB
      const int c = dw + DWV * i;                                      // wave-uniform
      if (allx || (!allw && c < XB)) {
        uint32_t o = vx0 + (uint32_t)i * sxs;
        if (tail && kb + st * BK + kc >= ke) o = kOOB;
        dma16s(rX, xd + c * 1024, o, sx);
      } else {
        const bool last = mayend && c >= NB;
        const int blk = last ? WB - 1 : c - XB;
        uint32_t o = last ? vlast : vwr + (uint32_t)(i - IW) * sws;
        if (wedge && n0 + blk * 8 >= p.N) o = kOOB;
        if (tail && kb + st * BK + (last ? kcl : kc) >= ke) o = kOOB;
        dma16s_nt(rW, wd + blk * 1024, o, sw);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  f32x4 acc[FW][FX], acce[EW > 0 ? EW : 1];
#pragma unroll
  for (int i = 0; i < FW; ++i)
#pragma unroll
    for (int j = 0; j < FX; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < (EW > 0 ? EW : 1); ++i) acce[i] = f32x4{0.f, 0.f, 0.f, 0.f};

#define OJX_KX_RD(sb, off) (*reinterpret_cast<const bf16x8*>((sb) + (off)))
  // groups: one per W fragment (position pp), FX MFMAs (+1 for the first EW); the last PD groups of a stage run
  // after the barrier that publishes the next stage, with their operands already in registers
  constexpr int PD = 2;
  constexpr int NMG = FW - PD;
  constexpr int H0 = (GPW + 1) / 2;           // DMAs right after the barrier
  constexpr int NDG = GPW - H0 < NMG - 2 ? GPW - H0 : (NMG - 2 > 0 ? NMG - 2 : 0);  // groups carrying one more
  constexpr int H1 = GPW - NDG;               // issued after the barrier (H0 plus what does not fit the groups)

  bf16x8 xc[NX], wr[PD + 1];
  static_assert((XD - 1) * GPW < 64, "DMA batches in flight must fit the vmcnt counter");
  if (nk > 0) {
#pragma unroll
    for (int st = 0; st < XD; ++st) dma(st, 0, GPW);
    if (dmaw) wait_vmcnt<(XD - 1) * GPW>();  // stage 0 has landed
    kx_barrier();
#pragma unroll
    for (int i = 0; i < NX; ++i) xc[i] = OJX_KX_RD(xring, xoff[i]);
#pragma unroll
    for (int d = 0; d < PD; ++d) wr[d] = OJX_KX_RD(wring, woff[d]);
    kx_barrier();       // every wave holds its x fragments of stage 0: x slot 0 is free
    dma(XD, 0, H1);
  }
  for (int t = 0; t < nk; ++t) {
    const uint8_t* sw = wring + (t % S::WD) * WST;
#pragma unroll
    for (int pp = 0; pp < NMG; ++pp) {
      wr[(pp + PD) % (PD + 1)] = OJX_KX_RD(sw, woff[pp + PD]);
      const bf16x8 a = wr[pp % (PD + 1)];
#pragma unroll
      for (int i = 0; i < FX; ++i) acc[pp][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, xc[i], acc[pp][i], 0, 0, 0);
      if constexpr (EW > 0)
        if (pp < EW) acce[pp] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, xc[FX], acce[pp], 0, 0, 0);
      if (pp < NDG) dma(t + XD, H1 + pp, H1 + pp + 1);
    }
    bf16x8 xn[NX], wn[PD];
    const bool more = t + 1 < nk;
    if (more) {
      if (dmaw) wait_vmcnt<(XD - 1) * GPW>();  // stage t+1 has landed (the batches of t+2 .. t+XD may not)
      kx_barrier();       // every wave's has, and every wave's W reads of stage t are done
      const uint8_t* nw = wring + ((t + 1) % S::WD) * WST;
      const uint8_t* nx = xring + ((t + 1) % XD) * XST;
#pragma unroll
      for (int i = 0; i < NX; ++i) xn[i] = OJX_KX_RD(nx, xoff[i]);
#pragma unroll
      for (int d = 0; d < PD; ++d) wn[d] = OJX_KX_RD(nw, woff[d]);
    }
#pragma unroll
    for (int pp = NMG; pp < FW; ++pp) {
      const bf16x8 a = wr[pp % (PD + 1)];
#pragma unroll
      for (int i = 0; i < FX; ++i) acc[pp][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, xc[i], acc[pp][i], 0, 0, 0);
      if constexpr (EW > 0)
        if (pp < EW) acce[pp] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, xc[FX], acce[pp], 0, 0, 0);
    }
    if (more) {
      kx_barrier();       // every wave holds its x fragments of stage t+1: that x slot takes stage t+1+XD
      dma(t + 1 + XD, 0, H1);
#pragma unroll
      for (int i = 0; i < NX; ++i) xc[i] = xn[i];
#pragma unroll
      for (int d = 0; d < PD; ++d) wr[d] = wn[d];
    }
  }
#undef OJX_KX_RD
  wait_vmcnt<0>();
  kx_barrier();  // LDS is free for the pair exchange

  // ------------------------------------------------------------------ pair reduction
  // Fragment f of a wave: acc[f / FX][f % FX] for f < FW FX, then acce[f - FW FX]. Wave g (h = 0) finishes
  // fragments 0 .. HF-1 and wave g+4 (h = 1) the rest. Two rounds through LDS (both halves at once would not fit):
  // wave g+4 hands over its first half, then wave g its second.
  float* const xch = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int round = 0; round < 2; ++round) {
    const int lo = round == 0 ? 0 : HF, hi = round == 0 ? HF : NACC;
    if (h != round) {  // the writer of this round
#pragma unroll
      for (int f = lo; f < hi; ++f) {
        const f32x4 v = f < FW * FX ? acc[f / FX][f % FX] : acce[f - FW * FX];
        *reinterpret_cast<f32x4*>(xch + ((g * HF + f - lo) * 64 + lane) * 4) = v;
      }
    }
    kx_barrier();
    if (h == round) {
#pragma unroll
      for (int f = lo; f < hi; ++f) {
        const f32x4 o = *reinterpret_cast<const f32x4*>(xch + ((g * HF + f - lo) * 64 + lane) * 4);
        if (f < FW * FX) acc[f / FX][f % FX] += o;
        else acce[f - FW * FX] += o;
      }
    }
    if (round == 0) kx_barrier();  // round 1 writes over the same LDS
  }

  // ------------------------------------------------------------------ epilogue
  if constexpr (EPI == EPI_FATTN) {
    static_assert(XE == 0, "the prep epilogue needs whole rows per SIMD group");
    if (h == 0) kx_fattn_epilogue<FW, FX, 0>(p, acc, g, lane, m0, n0, smem);
    else kx_fattn_epilogue<FW, FX, 1>(p, acc, g, lane, m0, n0, smem);
    return;
  }
  // lane holds v[e] = y[m][n + e]: m = m0 + 16 xf + lr, n = n0 + 16 wf + 4 lg
  if constexpr (EPI != EPI_F32) {
    if (p.one_launch) {  // this split's fp32 plane, then the tile's last split reduces (gemm_common.h)
      const __amdgpu_buffer_rsrc_t rsP = make_rsrc(p.ol_parts, (int64_t)p.splits * p.M * p.N * 4);
      const int64_t zo = (int64_t)z * p.M * p.N;
#pragma unroll
      for (int f = 0; f < NACC; ++f) {
        if ((f < HF) != (h == 0)) continue;
        const int wf = f < FW * FX ? wfrag(f / FX) : wfrag(f - FW * FX);
        const int xf = f < FW * FX ? g * FX + f % FX : xe;
        if (f >= FW * FX && wf < wnom) continue;  // stored by the neighbouring group
        const int m = m0 + xf * 16 + lr, n = n0 + wf * 16 + lg * 4;
        const f32x4 v = f < FW * FX ? acc[f / FX][f % FX] : acce[f - FW * FX];
        if (m < p.M && n < p.N)
          __builtin_amdgcn_raw_buffer_store_b128(v, rsP, (uint32_t)((zo + (int64_t)m * p.N + n) * 4), 0, kCoh);
      }
      // items batched per thread where the tile is small enough to keep the loads in registers
      ol_epilogue<BN, BM, 512, (BN * BM <= 144 * 128 ? 4 : 2)>(p, EPI, tn, tm, reinterpret_cast<float*>(smem));
      return;
    }
  }
#pragma unroll
  for (int f = 0; f < NACC; ++f) {
    if ((f < HF) != (h == 0)) continue;
    int wf, xf;
    bool keep = true;
    if (f < FW * FX) {
      wf = wfrag(f / FX);
      xf = g * FX + f % FX;
    } else {
      wf = wfrag(f - FW * FX);
      xf = xe;
      keep = wf >= wnom;  // extras that overlap the neighbouring group's are stored by that group
    }
    const f32x4 v = f < FW * FX ? acc[f / FX][f % FX] : acce[f - FW * FX];
    if (EPI == EPI_SILU) {
      const f32x4 u = shfl4(v, 16);  // every lane takes part in the exchange
      if (keep) store_silu_pair(p, m0 + xf * 16 + lr, n0 + wf * 16 + lg * 4, (lg & 1) == 0, v, u);
    } else if (keep) {
      store4(p, EPI, z, m0 + xf * 16 + lr, n0 + wf * 16 + lg * 4, true, v, v);
    }
  }
}

}  // namespace

template <int FW, int FX, int XE, int XD, int EPI>
__device__ __forceinline__ void kx_dir(const GemmParams& p) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (p.wpk) {
    if (XE == 2 && (wave & 1)) kx_body<FW, FX, XE, XD, EPI, true, true>(p);
    else kx_body<FW, FX, XE, XD, EPI, false, true>(p);
  } else {
    if (XE == 2 && (wave & 1)) kx_body<FW, FX, XE, XD, EPI, true, false>(p);
    else kx_body<FW, FX, XE, XD, EPI, false, false>(p);
  }
}

template <int FW, int FX, int XE, int XD>
__global__ void __launch_bounds__(512) gemm_kx_kernel(const GemmParams p, const int epi) {
  if constexpr (FW == 16 && XE == 0) {  // the 256-row tiles also carry the full-attention prep epilogue
    if (epi == EPI_FATTN) {
      kx_dir<FW, FX, XE, XD, EPI_FATTN>(p);
      return;
    }
  }
  if (epi == EPI_SILU) kx_dir<FW, FX, XE, XD, EPI_SILU>(p);
  else if (epi == EPI_RESID) kx_dir<FW, FX, XE, XD, EPI_RESID>(p);
  else if (epi == EPI_F32) kx_dir<FW, FX, XE, XD, EPI_F32>(p);
  else kx_dir<FW, FX, XE, XD, EPI_BF16>(p);
}

// Tile shapes of this family (registered in gemm.hip's tile table): BN x BM = 16 FW x 16 (4 FX + XE).
template __global__ void gemm_kx_kernel<9, 4, 2, 2>(const GemmParams, const int);  // 144 x 288
template __global__ void gemm_kx_kernel<8, 4, 2, 2>(const GemmParams, const int);  // 128 x 288
template __global__ void gemm_kx_kernel<9, 2, 1, 2>(const GemmParams, const int);  // 144 x 144
template __global__ void gemm_kx_kernel<8, 4, 0, 2>(const GemmParams, const int);  // 128 x 256
template __global__ void gemm_kx_kernel<9, 1, 0, 2>(const GemmParams, const int);  // 144 x 64
template __global__ void gemm_kx_kernel<9, 2, 0, 2>(const GemmParams, const int);  // 144 x 128
template __global__ void gemm_kx_kernel<8, 2, 0, 2>(const GemmParams, const int);  // 128 x 128
template __global__ void gemm_kx_kernel<8, 1, 0, 2>(const GemmParams, const int);  // 128 x 64
template __global__ void gemm_kx_kernel<16, 2, 0, 2>(const GemmParams, const int);  // 256 x 128: one head per tile
template __global__ void gemm_kx_kernel<16, 1, 0, 2>(const GemmParams, const int);  // 256 x 64
template __global__ void gemm_kx_kernel<10, 4, 0, 2>(const GemmParams, const int);  // 160 x 256
template __global__ void gemm_kx_kernel<10, 2, 0, 2>(const GemmParams, const int);  // 160 x 128
// a deeper ring for the weight-streaming M = 64-128: twice the bytes in flight per CU
template __global__ void gemm_kx_kernel<8, 1, 0, 4>(const GemmParams, const int);  // 128 x 64, 4 stages ahead

}  // namespace ojx
