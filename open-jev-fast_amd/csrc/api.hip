// C-ABI of libojx.so (declared in include/ojx.h): argument checks, plan lookup, and the launch sequences of the
// fused projection entry points.
#include "ojx_internal.h"
#include "ojx.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <mutex>
#include <string>

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return OJX_OK;
  return fail(OJX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t kchunk_for(int64_t K, int64_t S) { return cdiv(cdiv(K, S), 8) * 8; }
// split-K chunk over a packed weight: whole 64-k stages
inline int64_t kchunk_pk(int64_t K, int64_t S) { return cdiv(cdiv(K, S), 64) * 64; }
inline bool is_packed_kind(int32_t kind) { return (kind & OJX_KIND_PACKED) != 0; }

struct PlanEntry {
  int64_t M, N, K;
  int32_t kind, tile, splitk, tail_tile, tail_splitk, tail_rows, one_launch;
};

// Measured on MI355X by the offline sweep (tuning script in the package); shapes not listed use heuristic_plan.
const PlanEntry kPlan[] = {
#include "plan_table.inc"
};

constexpr int kSplits[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 16};
constexpr int kMaxSplit = 16;

constexpr int kSkMaxPieces = 64;  // gemm_sk.hip: pieces one stream-K tile may be split into
constexpr int kMaxGrid = 1024;    // persistent grid cap (one workgroup per CU)

bool is_sk(int32_t tile) {
  const ojx::TileInfo* t = ojx::tile_info(tile);
  return t != nullptr && t->family == 5;
}

// Compute units of the current device (the persistent grid size), cached per device.
int device_cus() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return std::min(cus[dev], kMaxGrid);
}

// Work split of the persistent stream-K family: whole-tile waves of `grid` workgroups over the first dp tiles,
// then the K iterations of the remaining R tiles shared by gs workgroups (at most S pieces per tile on average).
struct SkPlan {
  int grid, dp, gs;
  bool partial;        // some tile is split over several workgroups: partial slots are used
  int64_t slot_bytes;  // 2 gs partial tiles of fp32
};
SkPlan sk_plan(const ojx::TileInfo* t, int64_t M, int64_t N, int64_t K, int32_t S) {
  SkPlan sp{};
  const int64_t tiles = cdiv(N, t->bn) * cdiv(M, t->bm);
  const int64_t ipt = cdiv(K, t->bk);  // the family's K per stream-K iteration
  const int64_t G = device_cus();
  const int64_t dp = (tiles / G) * G, R = tiles - dp;
  int64_t gs = 0;
  if (R > 0) {
    gs = std::min(std::min(G, R * (int64_t)S), R * ipt);
    // keep every tile within kSkMaxPieces pieces: a tile spans at most (ipt - 1) / floor(T / gs) + 2 ranges
    while (gs > R && (ipt - 1) / ((R * ipt) / gs) + 2 > kSkMaxPieces) --gs;
  }
  sp.dp = (int)dp;
  sp.gs = (int)gs;
  sp.grid = (int)(dp > 0 ? G : std::max<int64_t>(gs, 1));
  sp.partial = gs > R;
  sp.slot_bytes = gs > R ? 2 * gs * (int64_t)t->bn * t->bm * 4 : 0;
  return sp;
}

bool part_fits(int64_t K, int32_t tile, int32_t splitk) {
  if (tile < 0 || tile >= ojx::num_tiles() || ojx::tile_info(tile)->family < 0) return false;  // < 0: retired id
  if (splitk < 1 || splitk > kMaxSplit) return false;
  if (is_sk(tile)) return true;  // splitk is the stream-K spread there, not a K split
  const int64_t ch = kchunk_for(K, splitk);
  return (splitk - 1) * ch < K;  // every split owns a non-empty K range
}

// Tile families that read the packed layout (without tails, with splits of whole 64-k stages): 0 (both operands
// through registers and LDS), 5 (persistent) and 6 (K-interleaved).
bool reads_packed(int32_t tile) {
  const ojx::TileInfo* t = ojx::tile_info(tile);
  return t != nullptr && (t->family == 0 || t->family == 5 || t->family == 6);
}

// A packed weight: no tails, splits of whole 64-k stages (the persistent family's splitk is its stream-K spread).
bool cfg_fits_packed(int64_t N, int64_t K, const ojx_cfg& c) {
  if (!reads_packed(c.tile) || c.tail_rows != 0 || c.splitk < 1 || c.splitk > kMaxSplit) return false;
  if (N % 16 != 0 || K % 64 != 0 || N * K * 2 >= (1LL << 31)) return false;
  if (is_sk(c.tile)) return true;
  return (c.splitk - 1) * kchunk_pk(K, c.splitk) < K;
}

// One-launch split-K: family 0 with a real split and no tail, within the counters and 32-bit plane offsets.
bool one_launch_fits(int64_t M, int64_t N, const ojx_cfg& c) {
  if (c.one_launch == 0) return true;
  const ojx::TileInfo* t = ojx::tile_info(c.tile);
  if (t == nullptr || c.splitk < 2 || c.tail_rows != 0) return false;
  // 1: the skinny family 0 or the K-interleaved family 6; 2 (the RMSNorm fold too): family 0 only
  if (!(c.one_launch == 1 && (t->family == 0 || t->family == 6)) && !(c.one_launch == 2 && t->family == 0))
    return false;
  const int64_t tm = cdiv(M > 0 ? M : 1, t->bm), tn = cdiv(N, t->bn);
  return tm * tn <= ojx::kOlMaxTiles && tm <= ojx::kOlMaxBlocks && (int64_t)c.splitk * M * N * 4 < (1LL << 31);
}

bool cfg_fits(int64_t M, int64_t N, int64_t K, const ojx_cfg& c, bool packed = false) {
  if (!one_launch_fits(M, N, c)) return false;
  if (packed) return cfg_fits_packed(N, K, c);
  if (!part_fits(K, c.tile, c.splitk)) return false;
  if (c.tail_rows == 0) return true;
  return c.tail_rows > 0 && c.tail_rows < N && c.tail_rows % 8 == 0 && part_fits(K, c.tail_tile, c.tail_splitk);
}

// The launches of a configuration: rows [0, N - tail_rows) with (tile, splitk), then the tail.
struct Part {
  ojx_cfg c;     // tile and split of this launch (no tail)
  int64_t n0, n; // W rows (output columns) it covers
  int64_t ws;    // byte offset of its split-K partials in the workspace
};
// Workspace of one launch: the stream-K partial slots, or the split-K fp32 planes.
int64_t part_ws_bytes(const ojx_cfg& c, int64_t M, int64_t n, int64_t K) {
  if (is_sk(c.tile)) {
    const SkPlan sp = sk_plan(ojx::tile_info(c.tile), M, n, K, c.splitk);
    return sp.slot_bytes;
  }
  if (c.one_launch) {  // the planes, then the per-tile row sums of squares
    const ojx::TileInfo* t = ojx::tile_info(c.tile);
    return cdiv((int64_t)c.splitk * M * n * 4, 256) * 256 + cdiv(cdiv(n, t->bn) * M * 4, 256) * 256;
  }
  return c.splitk > 1 ? cdiv((int64_t)c.splitk * M * n * 4, 256) * 256 : 0;
}
int split_parts(const ojx_cfg& c, int64_t M, int64_t N, int64_t K, Part out[2]) {
  const int64_t nt = c.tail_rows;
  out[0] = Part{ojx_cfg{c.tile, c.splitk, 0, 1, 0, c.one_launch}, 0, N - nt, 0};
  if (nt == 0) return 1;
  const int64_t ws0 = cdiv(part_ws_bytes(out[0].c, M, N - nt, K), 256) * 256;
  out[1] = Part{ojx_cfg{c.tail_tile, c.tail_splitk, 0, 1, 0}, N - nt, nt, ws0};
  return 2;
}
int64_t workspace_for(const ojx_cfg& c, int64_t M, int64_t N, int64_t K) {
  Part parts[2];
  const int np = split_parts(c, M, N, K, parts);
  return parts[np - 1].ws + part_ws_bytes(parts[np - 1].c, M, parts[np - 1].n, K);
}

ojx_cfg heuristic_plan(int64_t M, int64_t N, int64_t K, int32_t kind) {
  ojx_cfg c{};
  if (is_packed_kind(kind)) {  // skinny tile, K-interleaved tile or persistent tile for the M range
    c.tile = M <= 16 ? 0 : M <= 64 ? 84 : M <= 128 ? 85 : M <= 288 ? 80 : 73;
    const ojx::TileInfo* t = ojx::tile_info(c.tile);
    const int64_t tiles = cdiv(N, t->bn) * cdiv(M, t->bm);
    int64_t S = 1;
    while (S < 8 && tiles * S * 2 <= 320 && K / (S * 2) >= 512) S *= 2;
    c.splitk = (int32_t)S;
    while (c.splitk > 1 && !cfg_fits_packed(N, K, c)) --c.splitk;
    return c;
  }
  if (M <= 16) c.tile = 0;
  else if (M <= 32) c.tile = 2;
  else if (M <= 64) c.tile = 4;
  else if (M <= 128) c.tile = 6;
  else if (M <= 384) c.tile = 10;
  else c.tile = 7;
  const ojx::TileInfo* t = ojx::tile_info(c.tile);
  const int64_t tiles = cdiv(N, t->bn) * cdiv(M, t->bm);
  int64_t S = 1;
  while (S < 8 && tiles * S * 2 <= 512 && K / (S * 2) >= 512) S *= 2;
  c.splitk = (int32_t)S;
  return c;
}

int resolve(int64_t M, int64_t N, int64_t K, int32_t kind, const ojx_cfg* cfg, ojx_cfg* out) {
  if (cfg != nullptr) {
    if (!cfg_fits(M, N, K, *cfg, is_packed_kind(kind)))
      return fail(OJX_ERR_CONFIG, "config (tile %d, splitk %d, tail %d/%d/%d) invalid for M=%lld N=%lld K=%lld",
                  cfg->tile, cfg->splitk, cfg->tail_tile, cfg->tail_splitk, cfg->tail_rows, (long long)M,
                  (long long)N, (long long)K);
    *out = *cfg;
    return OJX_OK;
  }
  return ojx_plan(M, N, K, kind, out);
}

int check_dims(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N <= 0 || K <= 0) return fail(OJX_ERR_SHAPE, "bad shape M=%lld N=%lld K=%lld", (long long)M,
                                              (long long)N, (long long)K);
  if (M >= (1LL << 31) || N >= (1LL << 31) || K >= (1LL << 31))
    return fail(OJX_ERR_SHAPE, "shape dimension exceeds 2^31");
  if (N % 8 != 0 || K % 8 != 0)
    return fail(OJX_ERR_SHAPE, "N (%lld) and K (%lld) must be multiples of 8", (long long)N, (long long)K);
  return OJX_OK;
}

// One GEMM launch with the given tile / split count and epilogue.
// With hn_out (persistent family, residual epilogue, split tiles only): the split-tile pass is fused with the
// RMSNorm of the rows, writing h and hn.
int gemm(const ojx_cfg& c, int epi, const void* x, int64_t ldx, const void* w, int64_t ldw, void* out, int64_t ldo,
         const void* res, int64_t ldr, int64_t M, int64_t N, int64_t K, hipStream_t st, void* ws = nullptr,
         int64_t ws_off = 0, const float* w1 = nullptr, const int32_t* rowmask = nullptr, float eps = 0.f,
         uint16_t* hn_out = nullptr, bool packed = false, const ojx::FattnParams* fa = nullptr) {
  const ojx::TileInfo* t = ojx::tile_info(c.tile);
  ojx::GemmParams p;
  p.fa = fa != nullptr ? *fa : ojx::FattnParams{};
  p.W = static_cast<const uint16_t*>(w);
  p.ldw = ldw;
  p.X = static_cast<const uint16_t*>(x);
  p.ldx = ldx;
  p.out = out;
  p.ldo = ldo;
  p.res = static_cast<const uint16_t*>(res);
  p.ldr = ldr;
  p.part_stride = M * N;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.kchunk = (int)(packed ? kchunk_pk(K, c.splitk) : kchunk_for(K, c.splitk));
  p.wpk = packed ? 1 : 0;
  p.tiles_n = (int)cdiv(N, t->bn);
  p.tiles_m = (int)cdiv(M, t->bm);
  p.splits = c.splitk;
  p.sk_ws = nullptr;
  p.dp_tiles = 0;
  p.sk_grid = 0;
  p.one_launch = 0;
  p.ol_parts = nullptr;
  p.ol_ss = nullptr;
  p.w1 = w1;
  p.rowmask = rowmask;
  p.eps = eps;
  p.hn = nullptr;
  p.ol_tiles = p.ol_blocks = nullptr;
  if (c.one_launch && c.splitk > 1) {
    if (ws == nullptr) return fail(OJX_ERR_WORKSPACE, "one-launch split-K plan needs a workspace");
    const int rc = hip_check(ojx::ol_counters(st, &p.ol_tiles, &p.ol_blocks), "one-launch counters");
    if (rc != OJX_OK) return rc;
    p.one_launch = c.one_launch;
    p.ol_parts = reinterpret_cast<float*>(static_cast<char*>(ws) + ws_off);
    p.ol_ss = reinterpret_cast<float*>(static_cast<char*>(ws) + ws_off + cdiv((int64_t)c.splitk * M * N * 4, 256) * 256);
    p.hn = c.one_launch == 2 ? hn_out : nullptr;
  }
  int grid = 0;
  if (t->family == 5) {
    const SkPlan sp = sk_plan(t, M, N, K, c.splitk);
    p.splits = 1;
    p.dp_tiles = sp.dp;
    p.sk_grid = sp.gs;
    grid = sp.grid;
    if (sp.partial) {
      if (ws == nullptr) return fail(OJX_ERR_WORKSPACE, "stream-K plan needs a workspace");
      p.sk_ws = reinterpret_cast<float*>(static_cast<char*>(ws) + ws_off);
    }
  }
  if ((int64_t)p.tiles_n * p.tiles_m * p.splits >= (1LL << 31)) return fail(OJX_ERR_SHAPE, "grid too large");
  if (hn_out != nullptr && t->family == 5)
    return hip_check(ojx::launch_gemm_residual_rmsnorm_sk(c.tile, p, w1, rowmask, eps, hn_out, st, grid),
                     "gemm + row pass launch");
  return hip_check(ojx::launch_gemm(c.tile, epi, p, st, grid), "gemm launch");
}

int check_operands(const void* x, const void* w, int64_t ldx, int64_t ldw, int64_t K) {
  if (x == nullptr || w == nullptr) return fail(OJX_ERR_ARG, "null x or w");
  if (!aligned(x, 16) || !aligned(w, 16)) return fail(OJX_ERR_ARG, "x and w must be 16-byte aligned");
  if (ldx < K || ldw < K || ldx % 8 != 0 || ldw % 8 != 0)
    return fail(OJX_ERR_ARG, "row strides ldx=%lld ldw=%lld must be >= K and multiples of 8", (long long)ldx,
                (long long)ldw);
  return OJX_OK;
}

int check_ws(void* ws, int64_t ws_bytes, int64_t need) {
  if (need == 0) return OJX_OK;
  if (ws == nullptr || ws_bytes < need)
    return fail(OJX_ERR_WORKSPACE, "workspace of %lld bytes needed, %lld given", (long long)need,
                (long long)(ws == nullptr ? 0 : ws_bytes));
  if (!aligned(ws, 16)) return fail(OJX_ERR_ARG, "workspace must be 16-byte aligned");
  return OJX_OK;
}

int check_packed_shape_int(int64_t N, int64_t K) {
  if (N % 16 != 0 || K % 64 != 0)
    return fail(OJX_ERR_SHAPE, "packed weights need N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)", (long long)N,
                (long long)K);
  if (N * K * 2 >= (1LL << 31)) return fail(OJX_ERR_SHAPE, "packed weight larger than 2 GiB");
  return OJX_OK;
}

int check_rows(int64_t M, int64_t H) {
  if (M < 0 || H <= 0 || H % 8 != 0 || H / 8 > 1024)
    return fail(OJX_ERR_SHAPE, "row kernels need H %% 8 == 0 and H/8 <= 1024 (H=%lld)", (long long)H);
  if (M >= (1LL << 31)) return fail(OJX_ERR_SHAPE, "M exceeds 2^31");
  return OJX_OK;
}

#define OJX_TRY(expr)               \
  do {                              \
    const int rc_ = (expr);         \
    if (rc_ != OJX_OK) return rc_;  \
  } while (0)

// ------------------------------------------------------------------------------------- static scratch
// Device memory of ojx_gemm_residual_rmsnorm_noalloc: one array per GPU, held for the life of the process. In host
// code `scratch` is only a handle for the symbol lookup; kernels get the device address from hipGetSymbolAddress.
constexpr int64_t kScratchBytes = OJX_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The scratch array's address on the current device (looked up once per device, with that device current).
int scratch_ptr(void** out) {
  int dev = 0;
  OJX_TRY(hip_check(hipGetDevice(&dev), "hipGetDevice"));
  if (dev < 0 || dev >= kMaxDevices) return fail(OJX_ERR_ARG, "device %d out of range [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    OJX_TRY(hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
    if (p == nullptr) return fail(OJX_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return OJX_OK;
}

}  // namespace

extern "C" {

const char* ojx_last_error(void) { return g_err.c_str(); }
#ifndef OJX_SRC_DIGEST
#define OJX_SRC_DIGEST "unknown"
#endif
// The digest is a hash of the sources the library was compiled from (computed by the package's build script), so a
// caller can tell whether the loaded binary matches a source tree.
const char* ojx_version(void) { return "ojx 0.2 gfx950 src:" OJX_SRC_DIGEST; }

int ojx_init(void) {
  OJX_TRY(hip_check(ojx::init_tiles(), "kernel attribute setup"));
  void* p = nullptr;
  return scratch_ptr(&p);
}

int ojx_num_tiles(void) { return ojx::num_tiles(); }

int ojx_tile_info(int32_t tile, int32_t* info7) {
  const ojx::TileInfo* t = ojx::tile_info(tile);
  if (t == nullptr) return fail(OJX_ERR_CONFIG, "tile %d out of range [0, %d)", tile, ojx::num_tiles());
  if (info7 == nullptr) return fail(OJX_ERR_ARG, "null info");
  info7[0] = t->bn; info7[1] = t->bm; info7[2] = t->bk; info7[3] = t->wn; info7[4] = t->wm; info7[5] = t->threads;
  info7[6] = t->family;
  return OJX_OK;
}

int ojx_plan(int64_t M, int64_t N, int64_t K, int32_t kind, ojx_cfg* out) {
  if (out == nullptr) return fail(OJX_ERR_ARG, "null plan output");
  const int32_t base = kind & ~OJX_KIND_PACKED;
  if (base < OJX_KIND_PLAIN || base > OJX_KIND_RESIDUAL || (kind & ~(OJX_KIND_PACKED | 3)) != 0)
    return fail(OJX_ERR_ARG, "unknown kind %d", kind);
  const bool packed = is_packed_kind(kind);
  for (const PlanEntry& e : kPlan) {
    if (e.M == M && e.N == N && e.K == K && e.kind == kind) {
      ojx_cfg c{e.tile, e.splitk, e.tail_tile, e.tail_splitk, e.tail_rows, e.one_launch};
      if (c.tail_splitk == 0) c.tail_splitk = 1;
      if (cfg_fits(M, N, K, c, packed)) { *out = c; return OJX_OK; }
    }
  }
  *out = heuristic_plan(M, N, K, kind);
  if (!cfg_fits(M, N, K, *out, packed)) *out = ojx_cfg{out->tile, 1, 0, 1, 0};
  return OJX_OK;
}

static bool candidate_ok(int64_t M, int64_t N, int64_t K, const ojx_cfg& c, bool packed) {
  if (!cfg_fits(M, N, K, c, packed)) return false;
  const ojx::TileInfo* t = ojx::tile_info(c.tile);
  const int64_t mp = cdiv(M > 0 ? M : 1, 16) * 16;
  if (t->bm >= 2 * mp) return false;                   // more than half the x tile would be padding
  if (c.splitk > 1 && kchunk_for(K, c.splitk) < 256) return false;
  return true;
}

// Candidates: every (tile, split) that fits, and for the skinny family 0 with a split the one-launch variant too.
int ojx_num_candidates(int64_t M, int64_t N, int64_t K, int32_t kind) {
  const bool packed = is_packed_kind(kind);
  int n = 0;
  const int nol = (kind & ~OJX_KIND_PACKED) == OJX_KIND_RESIDUAL ? 3 : 2;  // the RMSNorm fold: residual only
  for (int t = 0; t < ojx::num_tiles(); ++t)
    for (int s : kSplits)
      for (int ol = 0; ol < nol; ++ol) n += candidate_ok(M, N, K, ojx_cfg{t, s, 0, 1, 0, ol}, packed) ? 1 : 0;
  return n;
}

int ojx_candidate(int64_t M, int64_t N, int64_t K, int32_t kind, int32_t idx, ojx_cfg* out) {
  const bool packed = is_packed_kind(kind);
  if (out == nullptr) return fail(OJX_ERR_ARG, "null candidate output");
  int n = 0;
  const int nol = (kind & ~OJX_KIND_PACKED) == OJX_KIND_RESIDUAL ? 3 : 2;
  for (int t = 0; t < ojx::num_tiles(); ++t)
    for (int s : kSplits)
      for (int ol = 0; ol < nol; ++ol)
        if (candidate_ok(M, N, K, ojx_cfg{t, s, 0, 1, 0, ol}, packed)) {
          if (n == idx) { *out = ojx_cfg{t, s, 0, 1, 0, ol}; return OJX_OK; }
          ++n;
        }
  return fail(OJX_ERR_CONFIG, "candidate index %d out of range [0, %d)", idx, n);
}

int64_t ojx_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t kind, const ojx_cfg* cfg) {
  ojx_cfg c{};
  if (resolve(M, N, K, kind, cfg, &c) != OJX_OK) return -1;
  return workspace_for(c, M, N, K);
}

int ojx_gemm_splitk_f32(const void* x, const void* w, float* parts, int64_t M, int64_t N, int64_t K, int64_t ldx,
                        int64_t ldw, int32_t S, int32_t tile, ojx_stream_t stream) {
  OJX_TRY(check_dims(M, N, K));
  if (M == 0) return OJX_OK;
  OJX_TRY(check_operands(x, w, ldx, ldw, K));
  if (parts == nullptr || !aligned(parts, 16)) return fail(OJX_ERR_ARG, "parts must be 16-byte aligned");
  ojx_cfg c{};
  if (tile < 0) {
    OJX_TRY(ojx_plan(M, N, K, OJX_KIND_RESIDUAL, &c));
    if (is_sk(c.tile)) c = heuristic_plan(M, N, K, OJX_KIND_RESIDUAL);  // that family writes no K planes
  } else {
    c.tile = tile;
  }
  if (is_sk(c.tile))
    return fail(OJX_ERR_CONFIG, "tile %d (persistent stream-K family) has no split-K planes", c.tile);
  c.splitk = S;
  c.one_launch = 0;  // planes out, no reduction
  if (!cfg_fits(M, N, K, c))
    return fail(OJX_ERR_CONFIG, "split-K S=%d (tile %d) invalid for K=%lld", S, c.tile, (long long)K);
  return gemm(c, ojx::EPI_F32, x, ldx, w, ldw, parts, N, nullptr, 0, M, N, K, static_cast<hipStream_t>(stream));
}

}  // extern "C"

static int gemm_bf16_impl(const void* x, const void* w, void* y, int64_t M, int64_t N, int64_t K, int64_t ldx,
                          int64_t ldw, int64_t ldy, void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg,
                          ojx_stream_t stream, bool packed) {
  OJX_TRY(check_dims(M, N, K));
  if (M == 0) return OJX_OK;  // an empty tensor may have a null data pointer
  OJX_TRY(check_operands(x, w, ldx, ldw, K));
  if (y == nullptr || !aligned(y, 8) || ldy < N || ldy % 4 != 0)
    return fail(OJX_ERR_ARG, "y must be 8-byte aligned with row stride >= N and a multiple of 4");
  ojx_cfg c{};
  OJX_TRY(resolve(M, N, K, OJX_KIND_PLAIN | (packed ? OJX_KIND_PACKED : 0), cfg, &c));
  OJX_TRY(check_ws(workspace, workspace_bytes, workspace_for(c, M, N, K)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  Part parts[2];
  const int np = split_parts(c, M, N, K, parts);
  for (int i = 0; i < np; ++i) {
    const Part& q = parts[i];
    const void* wq = static_cast<const uint16_t*>(w) + q.n0 * ldw;
    uint16_t* yq = static_cast<uint16_t*>(y) + q.n0;
    if (q.c.splitk == 1 || is_sk(q.c.tile) || q.c.one_launch) {
      OJX_TRY(gemm(q.c, ojx::EPI_BF16, x, ldx, wq, ldw, yq, ldy, nullptr, 0, M, q.n, K, st,
                   workspace, q.ws, nullptr, nullptr, 0.f, nullptr, packed));
      continue;
    }
    float* pp = reinterpret_cast<float*>(static_cast<char*>(workspace) + q.ws);
    OJX_TRY(gemm(q.c, ojx::EPI_F32, x, ldx, wq, ldw, pp, q.n, nullptr, 0, M, q.n, K, st, nullptr, 0, nullptr,
                 nullptr, 0.f, nullptr, packed));
    OJX_TRY(hip_check(ojx::launch_reduce_bf16(pp, q.c.splitk, M * q.n, yq, ldy, (int)M, (int)q.n, st),
                      "reduce launch"));
  }
  return OJX_OK;
}

static int gemm_silu_mul_impl(const void* x, const void* w_gu_packed, void* out, int64_t M, int64_t I, int64_t K,
                              void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg, ojx_stream_t stream,
                              bool packed) {
  if (I <= 0 || I % 4 != 0) return fail(OJX_ERR_SHAPE, "I (%lld) must be a positive multiple of 4", (long long)I);
  const int64_t N = 2 * I;
  OJX_TRY(check_dims(M, N, K));
  if (M == 0) return OJX_OK;
  OJX_TRY(check_operands(x, w_gu_packed, K, K, K));
  if (out == nullptr || !aligned(out, 8)) return fail(OJX_ERR_ARG, "out must be 8-byte aligned");
  ojx_cfg c{};
  OJX_TRY(resolve(M, N, K, OJX_KIND_SILU_MUL | (packed ? OJX_KIND_PACKED : 0), cfg, &c));
  OJX_TRY(check_ws(workspace, workspace_bytes, workspace_for(c, M, N, K)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  Part parts[2];
  const int np = split_parts(c, M, N, K, parts);
  for (int i = 0; i < np; ++i) {
    const Part& q = parts[i];
    const void* wq = static_cast<const uint16_t*>(w_gu_packed) + q.n0 * K;
    uint16_t* oq = static_cast<uint16_t*>(out) + q.n0 / 2;  // packed blocks of 8 rows give 4 output columns
    if (q.c.splitk == 1 || is_sk(q.c.tile) || q.c.one_launch) {
      OJX_TRY(gemm(q.c, ojx::EPI_SILU, x, K, wq, K, oq, I, nullptr, 0, M, q.n, K, st,
                   workspace, q.ws, nullptr, nullptr, 0.f, nullptr, packed));
      continue;
    }
    float* pp = reinterpret_cast<float*>(static_cast<char*>(workspace) + q.ws);
    OJX_TRY(gemm(q.c, ojx::EPI_F32, x, K, wq, K, pp, q.n, nullptr, 0, M, q.n, K, st, nullptr, 0, nullptr, nullptr,
                 0.f, nullptr, packed));
    OJX_TRY(hip_check(ojx::launch_reduce_silu(pp, q.c.splitk, M * q.n, oq, I, (int)M, (int)q.n, st),
                      "reduce launch"));
  }
  return OJX_OK;
}

static int gemm_residual_rmsnorm_impl(const void* x, const void* w, const void* residual, const float* w1,
                                      const int32_t* rowmask, float eps, void* h_out, void* hn_out, int64_t M,
                                      int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                                      const ojx_cfg* cfg, ojx_stream_t stream, bool packed) {
  OJX_TRY(check_dims(M, N, K));
  if (M == 0) return OJX_OK;
  OJX_TRY(check_operands(x, w, K, K, K));
  if (residual == nullptr || h_out == nullptr || !aligned(residual, 16) || !aligned(h_out, 16))
    return fail(OJX_ERR_ARG, "residual and h_out must be non-null and 16-byte aligned");
  if (hn_out != nullptr) {
    OJX_TRY(check_rows(M, N));
    if (w1 == nullptr || !aligned(w1, 16) || !aligned(hn_out, 16))
      return fail(OJX_ERR_ARG, "w1 and hn_out must be non-null and 16-byte aligned");
  }
  if (M == 0) return OJX_OK;
  ojx_cfg c{};
  OJX_TRY(resolve(M, N, K, OJX_KIND_RESIDUAL | (packed ? OJX_KIND_PACKED : 0), cfg, &c));
  if (c.tail_rows != 0)
    return fail(OJX_ERR_CONFIG, "tail configurations apply to the plain and SiLU.mul GEMMs only (the RMSNorm "
                                "epilogue needs whole rows)");
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint16_t* h = static_cast<uint16_t*>(h_out);
  uint16_t* hn = static_cast<uint16_t*>(hn_out);
  if (c.one_launch && c.splitk > 1) {
    // one_launch 2: GEMM, split reduction, residual and RMSNorm in one launch; 1: the GEMM launch ends with h, and
    // the RMSNorm is a second launch over h (instead of over the S fp32 planes)
    OJX_TRY(check_ws(workspace, workspace_bytes, workspace_for(c, M, N, K)));
    OJX_TRY(gemm(c, ojx::EPI_RESID, x, K, w, K, h_out, N, residual, N, M, N, K, st, workspace, 0, w1, rowmask, eps,
                 hn, packed));
    if (hn == nullptr || c.one_launch == 2) return OJX_OK;
    return hip_check(ojx::launch_add_rmsnorm(h, nullptr, nullptr, 0, 0, w1, rowmask, eps, nullptr, hn, (int)M,
                                             (int)N, st), "rmsnorm launch");
  }
  if (c.splitk == 1 || is_sk(c.tile)) {
    OJX_TRY(check_ws(workspace, workspace_bytes, workspace_for(c, M, N, K)));
    if (hn != nullptr && is_sk(c.tile) && sk_plan(ojx::tile_info(c.tile), M, N, K, c.splitk).partial) {
      // persistent plan with split tiles: GEMM, then one launch that sums the pieces, adds the residual and
      // normalises each row
      return gemm(c, ojx::EPI_RESID, x, K, w, K, h_out, N, residual, N, M, N, K, st, workspace, 0, w1, rowmask,
                  eps, hn, packed);
    }
    OJX_TRY(gemm(c, ojx::EPI_RESID, x, K, w, K, h_out, N, residual, N, M, N, K, st, workspace, 0, nullptr, nullptr,
                 0.f, nullptr, packed));
    if (hn == nullptr) return OJX_OK;
    return hip_check(ojx::launch_add_rmsnorm(h, nullptr, nullptr, 0, 0, w1, rowmask, eps, nullptr, hn, (int)M,
                                             (int)N, st), "rmsnorm launch");
  }
  if (hn == nullptr && N / 8 > 1024) return fail(OJX_ERR_SHAPE, "split-K residual needs N/8 <= 1024");
  OJX_TRY(check_ws(workspace, workspace_bytes, workspace_for(c, M, N, K)));
  float* parts = static_cast<float*>(workspace);
  OJX_TRY(gemm(c, ojx::EPI_F32, x, K, w, K, parts, N, nullptr, 0, M, N, K, st, nullptr, 0, nullptr, nullptr, 0.f,
               nullptr, packed));
  return hip_check(ojx::launch_add_rmsnorm(static_cast<const uint16_t*>(residual), nullptr, parts, c.splitk, M * N,
                                           w1, rowmask, eps, h, hn, (int)M, (int)N, st), "rmsnorm launch");
}

extern "C" {

int ojx_gemm_bf16(const void* x, const void* w, void* y, int64_t M, int64_t N, int64_t K, int64_t ldx,
                  int64_t ldw, int64_t ldy, void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg,
                  ojx_stream_t stream) {
  return gemm_bf16_impl(x, w, y, M, N, K, ldx, ldw, ldy, workspace, workspace_bytes, cfg, stream, false);
}

int ojx_gemm_silu_mul(const void* x, const void* w_gu_packed, void* out, int64_t M, int64_t I, int64_t K,
                      void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg, ojx_stream_t stream) {
  return gemm_silu_mul_impl(x, w_gu_packed, out, M, I, K, workspace, workspace_bytes, cfg, stream, false);
}

int ojx_gemm_residual_rmsnorm(const void* x, const void* w, const void* residual, const float* w1,
                              const int32_t* rowmask, float eps, void* h_out, void* hn_out, int64_t M, int64_t N,
                              int64_t K, void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg,
                              ojx_stream_t stream) {
  return gemm_residual_rmsnorm_impl(x, w, residual, w1, rowmask, eps, h_out, hn_out, M, N, K, workspace,
                                    workspace_bytes, cfg, stream, false);
}

static int check_packed_shape(int64_t N, int64_t K) { return check_packed_shape_int(N, K); }

int ojx_pack_weight(const void* w, void* wp, int64_t N, int64_t K, ojx_stream_t stream) {
  OJX_TRY(check_dims(1, N, K));
  OJX_TRY(check_packed_shape(N, K));
  if (w == nullptr || wp == nullptr || !aligned(w, 16) || !aligned(wp, 16))
    return fail(OJX_ERR_ARG, "w and wp must be non-null and 16-byte aligned");
  return hip_check(ojx::launch_pack_weight(static_cast<const uint16_t*>(w), static_cast<uint16_t*>(wp), N, K,
                                           static_cast<hipStream_t>(stream)), "pack launch");
}

int ojx_unsplit_weight(const void* wsk, void* w, int64_t N, int64_t K, int64_t S, ojx_stream_t stream) {
  OJX_TRY(check_dims(1, N, K));
  if (S < 1 || K % S != 0) return fail(OJX_ERR_SHAPE, "K=%lld is not a multiple of S=%lld", (long long)K, (long long)S);
  if (wsk == nullptr || w == nullptr || !aligned(wsk, 16) || !aligned(w, 16))
    return fail(OJX_ERR_ARG, "wsk and w must be non-null and 16-byte aligned");
  if (K > 65535 * 64LL) return fail(OJX_ERR_SHAPE, "K=%lld too large (at most %lld)", (long long)K, 65535 * 64LL);
  return hip_check(ojx::launch_unsplit_weight(static_cast<const uint16_t*>(wsk), static_cast<uint16_t*>(w), K, N,
                                              static_cast<hipStream_t>(stream)), "unsplit launch");
}

int ojx_gemm_bf16_pk(const void* x, const void* wp, void* y, int64_t M, int64_t N, int64_t K, int64_t ldx,
                     int64_t ldy, void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg, ojx_stream_t stream) {
  OJX_TRY(check_packed_shape(N, K));
  return gemm_bf16_impl(x, wp, y, M, N, K, ldx, K, ldy, workspace, workspace_bytes, cfg, stream, true);
}

int ojx_gemm_silu_mul_pk(const void* x, const void* w_gu_pk, void* out, int64_t M, int64_t I, int64_t K,
                         void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg, ojx_stream_t stream) {
  OJX_TRY(check_packed_shape(2 * I, K));
  return gemm_silu_mul_impl(x, w_gu_pk, out, M, I, K, workspace, workspace_bytes, cfg, stream, true);
}

int ojx_gemm_residual_rmsnorm_pk(const void* x, const void* wp, const void* residual, const float* w1,
                                 const int32_t* rowmask, float eps, void* h_out, void* hn_out, int64_t M, int64_t N,
                                 int64_t K, void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg,
                                 ojx_stream_t stream) {
  OJX_TRY(check_packed_shape(N, K));
  return gemm_residual_rmsnorm_impl(x, wp, residual, w1, rowmask, eps, h_out, hn_out, M, N, K, workspace,
                                    workspace_bytes, cfg, stream, true);
}

static int check_fattn(int64_t N, int32_t HQ, int32_t HKV, int32_t D, int32_t RD, const float* qw1,
                       const float* kw1, const void* cosb, const void* sinb, const void* qt, const void* kt,
                       const void* vt, const void* gate) {
  if (D != 256) return fail(OJX_ERR_SHAPE, "full-attention prep supports head_dim 256 (D=%d)", D);
  if (HQ < 1 || HKV < 1 || HQ > 4096 || HKV > 4096) return fail(OJX_ERR_SHAPE, "bad head counts HQ=%d HKV=%d", HQ, HKV);
  if (RD < 16 || RD > D || RD % 16 != 0 || ((RD / 16) & (RD / 16 - 1)) != 0)
    return fail(OJX_ERR_SHAPE, "rotary dims RD=%d must be 16 * a power of two, <= D", RD);
  if (N < 0 || N * ((HQ + 2 * HKV + 3) / 4) >= (1LL << 31)) return fail(OJX_ERR_SHAPE, "bad token count");
  if (N == 0) return OJX_OK;  // nothing is read or written
  const void* ptrs[] = {qw1, kw1, cosb, sinb, qt, kt, vt, gate};
  for (const void* q : ptrs)
    if (q == nullptr || !aligned(q, 16)) return fail(OJX_ERR_ARG, "prep operands must be non-null, 16-byte aligned");
  return OJX_OK;
}

int ojx_fullattn_prep(const void* proj, int64_t N, int32_t HQ, int32_t HKV, int32_t D, int32_t RD, float eps,
                      const float* qw1, const float* kw1, const void* cosb, const void* sinb, void* qt, void* kt,
                      void* vt, void* gate, ojx_stream_t stream) {
  OJX_TRY(check_fattn(N, HQ, HKV, D, RD, qw1, kw1, cosb, sinb, qt, kt, vt, gate));
  if (N == 0) return OJX_OK;
  if (proj == nullptr || !aligned(proj, 16)) return fail(OJX_ERR_ARG, "proj must be non-null, 16-byte aligned");
  return hip_check(ojx::launch_fullattn_prep(static_cast<const uint16_t*>(proj), N, HQ, HKV, RD, eps, qw1, kw1,
                                             static_cast<const uint16_t*>(cosb), static_cast<const uint16_t*>(sinb),
                                             static_cast<uint16_t*>(qt), static_cast<uint16_t*>(kt),
                                             static_cast<uint16_t*>(vt), static_cast<uint16_t*>(gate),
                                             static_cast<hipStream_t>(stream)), "prep launch");
}

int ojx_gemm_qkv_fullattn_prep(const void* x, const void* w, int32_t w_packed, const float* qw1, const float* kw1,
                               const void* cosb, const void* sinb, void* qt, void* kt, void* vt, void* gate,
                               int64_t M, int64_t K, int32_t HQ, int32_t HKV, int32_t D, int32_t RD, float eps,
                               ojx_stream_t stream) {
  OJX_TRY(check_fattn(M, HQ, HKV, D, RD, qw1, kw1, cosb, sinb, qt, kt, vt, gate));
  if (RD != 64) return fail(OJX_ERR_SHAPE, "the fused prep epilogue supports RD = 64 (RD=%d)", RD);
  const int64_t N = (int64_t)(2 * HQ + 2 * HKV) * D;
  OJX_TRY(check_dims(M, N, K));
  if (M == 0) return OJX_OK;
  OJX_TRY(check_operands(x, w, K, K, K));
  if (w_packed) OJX_TRY(check_packed_shape_int(N, K));
  ojx_cfg c{M <= 64 ? 89 : 88, 1, 0, 1, 0};  // 256-row tiles: one head block each, no split (the norm needs sums)
  ojx::FattnParams fa{qw1, kw1, static_cast<const uint16_t*>(cosb), static_cast<const uint16_t*>(sinb),
                      static_cast<uint16_t*>(qt), static_cast<uint16_t*>(kt), static_cast<uint16_t*>(vt),
                      static_cast<uint16_t*>(gate), HQ, HKV, RD, eps};
  return gemm(c, ojx::EPI_FATTN, x, K, w, K, nullptr, 0, nullptr, 0, M, N, K, static_cast<hipStream_t>(stream),
              nullptr, 0, nullptr, nullptr, 0.f, nullptr, w_packed != 0, &fa);
}

int ojx_linattn_prep(const void* proj, const int32_t* hist, const int32_t* rep_ptr, const int32_t* rep_pos,
                     int64_t N, int64_t R, int64_t L2, const void* convw, const void* A_log, const void* dt_bias,
                     int32_t KD, int32_t VD, int32_t HV, int32_t HK, int32_t HD, int32_t rep_qk, void* q, void* k,
                     void* v, float* g, void* beta, ojx_stream_t stream) {
  if (HD != 128) return fail(OJX_ERR_SHAPE, "linear-attention prep supports head_dim 128 (HD=%d)", HD);
  if (HK < 1 || HK * HD != KD) return fail(OJX_ERR_SHAPE, "KD=%d must be HK * HD (HK=%d)", KD, HK);
  if (HV < 1 || HV > 256 || VD < 8 || VD % 8 != 0)
    return fail(OJX_ERR_SHAPE, "bad value dims VD=%d HV=%d (HV <= 256, VD a multiple of 8)", VD, HV);
  const int rq = rep_qk ? HV / HK : 1;
  if (rq != 1 && rq != 3) return fail(OJX_ERR_SHAPE, "replicated q/k needs HV / HK = 3 (HV=%d HK=%d)", HV, HK);
  if (N < 0 || N >= (1LL << 31) - 1 || R < 0 || R >= (1LL << 31) || L2 < 1 || R % L2 != 0)
    return fail(OJX_ERR_SHAPE, "bad sizes N=%lld R=%lld L2=%lld (R a multiple of L2)", (long long)N, (long long)R,
                (long long)L2);
  if (2 * KD + VD > 28672)  // the finished row is held in LDS (2 bytes per conv channel)
    return fail(OJX_ERR_SHAPE, "2 KD + VD = %d conv channels exceed 28672", 2 * KD + VD);
  if (R == 0) return OJX_OK;
  const void* ptrs[] = {proj, hist, rep_ptr, rep_pos, convw, A_log, dt_bias, q, k, v, g, beta};
  for (const void* p : ptrs)
    if (p == nullptr) return fail(OJX_ERR_ARG, "linear-attention prep operands must be non-null");
  const void* vec[] = {proj, hist, convw, q, k, v};
  for (const void* p : vec)
    if (!aligned(p, 16)) return fail(OJX_ERR_ARG, "proj, hist, convw, q, k and v must be 16-byte aligned");
  return hip_check(ojx::launch_linattn_prep(static_cast<const uint16_t*>(proj), hist, rep_ptr, rep_pos, N, R,
                                            static_cast<const uint16_t*>(convw), static_cast<const uint16_t*>(A_log),
                                            static_cast<const uint16_t*>(dt_bias), KD, VD, HV, rq,
                                            static_cast<uint16_t*>(q), static_cast<uint16_t*>(k),
                                            static_cast<uint16_t*>(v), g, static_cast<uint16_t*>(beta),
                                            static_cast<hipStream_t>(stream)), "linear-attention prep launch");
}

int ojx_gemm_residual_rmsnorm_noalloc(const void* x, const void* w, const void* residual, const float* w1,
                                      const int32_t* rowmask, float eps, void* h_out, void* hn_out, int64_t M,
                                      int64_t N, int64_t K, const ojx_cfg* cfg, ojx_stream_t stream) {
  OJX_TRY(check_dims(M, N, K));
  if (M == 0) return OJX_OK;
  ojx_cfg c{};
  OJX_TRY(resolve(M, N, K, OJX_KIND_RESIDUAL, cfg, &c));
  int64_t need = workspace_for(c, M, N, K);
  if (cfg != nullptr && need > kScratchBytes)
    return fail(OJX_ERR_WORKSPACE, "config (tile %d, splitk %d) needs %lld bytes of workspace; the static scratch of "
                "the allocation-free entry point holds %lld", c.tile, c.splitk, (long long)need,
                (long long)kScratchBytes);
  // The plan's own configuration, with its split-K count (or stream-K spread) lowered to the largest value that
  // is valid for the shape and whose workspace fits; `need` always belongs to the configuration in `c`.
  for (ojx_cfg t = c; need > kScratchBytes && t.splitk > 1;) {
    --t.splitk;
    if (!cfg_fits(M, N, K, t)) continue;
    const int64_t nt = workspace_for(t, M, N, K);
    if (nt <= kScratchBytes) {
      c = t;
      need = nt;
    }
  }
  if (need > kScratchBytes)
    return fail(OJX_ERR_WORKSPACE, "M=%lld N=%lld K=%lld needs %lld bytes of workspace, more than the static scratch "
                "(%lld)", (long long)M, (long long)N, (long long)K, (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  OJX_TRY(scratch_ptr(&ws));
  return ojx_gemm_residual_rmsnorm(x, w, residual, w1, rowmask, eps, h_out, hn_out, M, N, K, ws, kScratchBytes, &c,
                                   stream);
}

int ojx_add_rmsnorm(const void* x, const void* delta, const float* w1, const int32_t* rowmask, float eps,
                    void* h_out, void* hn_out, int64_t M, int64_t H, ojx_stream_t stream) {
  OJX_TRY(check_rows(M, H));
  if (M == 0) return OJX_OK;
  if (x == nullptr || hn_out == nullptr || w1 == nullptr) return fail(OJX_ERR_ARG, "null x, hn_out or w1");
  if (delta != nullptr && h_out == nullptr) return fail(OJX_ERR_ARG, "h_out required when delta is given");
  if (!aligned(x, 16) || !aligned(hn_out, 16) || !aligned(w1, 16) || (delta && !aligned(delta, 16)) ||
      (h_out && !aligned(h_out, 16)))
    return fail(OJX_ERR_ARG, "row kernel operands must be 16-byte aligned");
  if (M == 0) return OJX_OK;
  return hip_check(ojx::launch_add_rmsnorm(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(delta),
                                           nullptr, 0, 0, w1, rowmask, eps,
                                           delta ? static_cast<uint16_t*>(h_out) : nullptr,
                                           static_cast<uint16_t*>(hn_out), (int)M, (int)H,
                                           static_cast<hipStream_t>(stream)), "rmsnorm launch");
}

int ojx_add_rmsnorm_sk(const void* x, const float* parts, int32_t S, const float* w1, const int32_t* rowmask,
                       float eps, void* h_out, void* hn_out, int64_t M, int64_t H, ojx_stream_t stream) {
  OJX_TRY(check_rows(M, H));
  if (S < 1 || S > kMaxSplit) return fail(OJX_ERR_CONFIG, "S must be in [1, %d]", kMaxSplit);
  if (M == 0) return OJX_OK;
  if (x == nullptr || parts == nullptr || h_out == nullptr || hn_out == nullptr || w1 == nullptr)
    return fail(OJX_ERR_ARG, "null operand");
  if (!aligned(x, 16) || !aligned(parts, 16) || !aligned(h_out, 16) || !aligned(hn_out, 16) || !aligned(w1, 16))
    return fail(OJX_ERR_ARG, "row kernel operands must be 16-byte aligned");
  if (M == 0) return OJX_OK;
  return hip_check(ojx::launch_add_rmsnorm(static_cast<const uint16_t*>(x), nullptr, parts, S, M * H, w1, rowmask,
                                           eps, static_cast<uint16_t*>(h_out), static_cast<uint16_t*>(hn_out),
                                           (int)M, (int)H, static_cast<hipStream_t>(stream)), "rmsnorm launch");
}

static int silu_common(const void* gu, const void* tab, void* out, int64_t M, int64_t I, ojx_stream_t stream) {
  if (I <= 0 || I % 8 != 0 || M < 0) return fail(OJX_ERR_SHAPE, "silu_mul needs I %% 8 == 0 (I=%lld)", (long long)I);
  if (M == 0) return OJX_OK;
  if (gu == nullptr || out == nullptr || !aligned(gu, 16) || !aligned(out, 16))
    return fail(OJX_ERR_ARG, "gu and out must be non-null and 16-byte aligned");
  if (M == 0) return OJX_OK;
  return hip_check(ojx::launch_silu_mul(static_cast<const uint16_t*>(gu), static_cast<const uint16_t*>(tab),
                                        static_cast<uint16_t*>(out), (int)M, (int)I,
                                        static_cast<hipStream_t>(stream)), "silu_mul launch");
}

int ojx_silu_mul(const void* gu, void* out, int64_t M, int64_t I, ojx_stream_t stream) {
  return silu_common(gu, nullptr, out, M, I, stream);
}

int ojx_silu_mul_lut(const void* gu, const void* tab, void* out, int64_t M, int64_t I, ojx_stream_t stream) {
  if (tab == nullptr) return fail(OJX_ERR_ARG, "null table");
  return silu_common(gu, tab, out, M, I, stream);
}

int ojx_head_scores(const void* hn, int64_t rows, int64_t H, const int64_t* lastidx, int64_t R, const float* w,
                    const float* bias, float* scores, ojx_stream_t stream) {
  if (R < 0 || rows < 0 || H <= 0 || H % 8 != 0)
    return fail(OJX_ERR_SHAPE, "head needs H %% 8 == 0 (H=%lld), R, rows >= 0", (long long)H);
  if (R == 0) return OJX_OK;
  if (hn == nullptr || lastidx == nullptr || w == nullptr || scores == nullptr)
    return fail(OJX_ERR_ARG, "null hn, lastidx, w or scores");
  if (!aligned(hn, 16) || !aligned(w, 16) || !aligned(lastidx, 8) || !aligned(scores, 4))
    return fail(OJX_ERR_ARG, "hn and w must be 16-byte aligned, lastidx 8-byte aligned");
  return hip_check(ojx::launch_head_gemv(static_cast<const uint16_t*>(hn), rows, lastidx, R, w, bias, scores, (int)H,
                                         static_cast<hipStream_t>(stream)), "head launch");
}

int ojx_act_tables(void* silu_b, float* sig_f, ojx_stream_t stream) {
  if (silu_b == nullptr || sig_f == nullptr) return fail(OJX_ERR_ARG, "null table output");
  return hip_check(ojx::launch_act_tables(static_cast<uint16_t*>(silu_b), sig_f, static_cast<hipStream_t>(stream)),
                   "act_tables launch");
}

int ojx_pack_gate_up(const void* gate, const void* up, void* packed, int64_t I, int64_t K, ojx_stream_t stream) {
  if (I <= 0 || I % 4 != 0 || K <= 0 || K % 8 != 0)
    return fail(OJX_ERR_SHAPE, "pack_gate_up needs I %% 4 == 0 and K %% 8 == 0");
  if (gate == nullptr || up == nullptr || packed == nullptr || !aligned(gate, 16) || !aligned(up, 16) ||
      !aligned(packed, 16))
    return fail(OJX_ERR_ARG, "gate, up and packed must be non-null and 16-byte aligned");
  return hip_check(ojx::launch_pack_gate_up(static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up),
                                            static_cast<uint16_t*>(packed), (int)I, (int)K,
                                            static_cast<hipStream_t>(stream)), "pack launch");
}

}  // extern "C"
