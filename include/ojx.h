/*
 * ojx — MI355X (gfx950) dense bf16 projection kernels for the open-jev-fast 27B hybrid forward.
 *
 * C-ABI of libojx.so: plain C, raw device pointers, element counts and a HIP stream handle; no torch types.
 * All bf16 tensors are raw 16-bit patterns, row-major. A projection computes
 *     y[M,N] = x[M,K] . W[N,K]^T      (bf16 inputs, fp32 accumulation, bf16 output)
 * with both x and W K-contiguous, the layout of the reference's lt_matmul (src/lt.cpp:22-29) and F.linear.
 *
 * Every entry point returns OJX_OK (0) or an error code; ojx_last_error() gives the message of the last failure
 * on the calling thread. Launches go on the given stream, never synchronize and never allocate, so they can be
 * captured into a HIP graph. Entry points that take a workspace need ojx_workspace_bytes() bytes of device memory
 * there (0 bytes when the plan has no split-K and no stream-K partial tiles). A workspace is scratch for one call:
 * its contents on entry do not matter, and two calls that may run at the same time need separate workspaces.
 *
 * Global state (the plan table, kernel attributes) is read-only after the first call; concurrent calls on
 * different streams are safe as long as they do not share output or workspace buffers.
 */
#ifndef OJX_H
#define OJX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ojx_stream_t; /* hipStream_t; NULL = the null stream */

enum {
  OJX_OK = 0,
  OJX_ERR_ARG = 1,       /* null / misaligned pointer, bad stride */
  OJX_ERR_SHAPE = 2,     /* unsupported shape (e.g. N or K not a multiple of 8, H/8 > 1024) */
  OJX_ERR_WORKSPACE = 3, /* workspace missing or too small for the plan */
  OJX_ERR_CONFIG = 4,    /* tile id / split-K count out of range */
  OJX_ERR_HIP = 5        /* a HIP runtime call failed */
};

enum {
  OJX_KIND_PLAIN = 0,     /* y = x W^T */
  OJX_KIND_SILU_MUL = 1,  /* gate-up projection with the SiLU(gate) * up epilogue */
  OJX_KIND_RESIDUAL = 2,  /* out / o_proj / down projection with residual add (+ RMSNorm) */
  OJX_KIND_PACKED = 4     /* or-ed into a kind: the weight is in the ojx_pack_weight layout (the *_pk entry points) */
};

/* One kernel configuration: a tile shape from the tile registry and a split-K count. Optionally the last
 * tail_rows rows of W (outputs N - tail_rows .. N - 1) run as a second launch with their own tile and split: when
 * N / BN tiles leave a few tiles over a whole number of rounds on the 256 CUs, a finer tile for the remainder
 * replaces a second, mostly idle round. tail_rows = 0 (the zero-initialised default) means no tail; tails apply
 * to ojx_gemm_bf16 and ojx_gemm_silu_mul (tail_rows a multiple of 8 there).
 * one_launch = 1 (tile families 0 and 6, splitk >= 2, no tail): the split-K reduction and its epilogue run in the
 * GEMM launch itself (the last split of each tile to finish sums the fp32 planes, in split order); for
 * ojx_gemm_residual_rmsnorm the launch ends with h and a second launch normalises h (instead of reading the
 * planes). one_launch = 2 (family 0, ojx_gemm_residual_rmsnorm): the RMSNorm too (the last tile of each row block
 * to finish normalises its rows): one launch instead of two. Results equal the two-launch path's bit for bit,
 * except hn under one_launch = 2, whose sum of squares is added in another order (one rounding step at most). The
 * arrival counters are the library's (zero at load, left zero by every call), one set per stream for the first 8
 * streams of a device that launch such a plan: calls on different streams (each with its own workspace) may
 * overlap; streams past the 8th share sets, and overlapping calls on a shared set race, as do graph replays on a
 * stream other than the capture stream. */
typedef struct {
  int32_t tile;
  int32_t splitk;
  int32_t tail_tile;
  int32_t tail_splitk;
  int32_t tail_rows;
  int32_t one_launch;
} ojx_cfg;

const char* ojx_last_error(void);
/* "ojx <version> gfx950 src:<digest>": the digest hashes the sources the library was built from. */
const char* ojx_version(void);

/* Sets kernel attributes on the current device. Optional: every launch does it on first use. */
int ojx_init(void);

/* Tile registry: info7 = {BN (W rows), BM (x rows), BK, waves along N, waves along M, threads, family}.
 * Family (all on 16x16x32 MFMA): 0 both operands through registers into LDS; 5 persistent (one workgroup per CU,
 * two waves per SIMD, LDS DMA): whole-tile waves, then the remaining tiles' K iterations spread over the grid
 * (stream-K), with splitk = the most pieces one remaining tile is cut into on average (1 = whole tiles), split
 * tiles summed by a second, small launch; 6 K-interleaved wave pairs (the two waves of a SIMD take alternate
 * 32-k halves and add their sums at the end); -1 a retired id (ids 16-72), which no plan, candidate list or
 * launch accepts.
 * Tiles of families 0 and 5 sum K in the same order, so without split-K (stream-K spread 1 for family 5) they
 * give bit-identical results; family 6 agrees with them to fp32 rounding. Stream-K results are deterministic:
 * the pieces of a tile are summed in K order whatever order they finish in. */
int ojx_num_tiles(void);
int ojx_tile_info(int32_t tile, int32_t* info7);

/* Plan lookup for a shape: a static table measured offline on MI355X, with a heuristic for shapes not in it.
 * Never times anything, so it is safe during graph capture.
 * Replaces the per-shape cuBLASLt heuristic/search: lt_setup (src/lt.cpp:15-42), _tune (src/fastmodel.py:114-132),
 * lt2_plan / lt2_search (src/lt.cpp:64-159). For OJX_KIND_SILU_MUL, N is the packed 2*I. */
int ojx_plan(int64_t M, int64_t N, int64_t K, int32_t kind, ojx_cfg* out);

/* Candidate configurations for a shape (every tile x split-K that is valid), the list a tuner sweeps.
 * Mirrors lt_setup's algorithm count and lt_matmul's algorithm index (src/lt.cpp:15-55). */
int ojx_num_candidates(int64_t M, int64_t N, int64_t K, int32_t kind);
int ojx_candidate(int64_t M, int64_t N, int64_t K, int32_t kind, int32_t idx, ojx_cfg* out);

/* Workspace bytes the call needs with cfg (NULL = the plan's choice). */
int64_t ojx_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t kind, const ojx_cfg* cfg);

/* y[M,N] (row stride ldy) = x[M,K] (row stride ldx) . W[N,K]^T (row stride ldw).
 * Replaces lt_matmul (src/lt.cpp:43-55) / F.linear as called by _mm (src/fastmodel.py:168-175).
 * N, K, ldx, ldw multiples of 8; ldy a multiple of 4. cfg NULL = the plan's choice. */
int ojx_gemm_bf16(const void* x, const void* w, void* y, int64_t M, int64_t N, int64_t K, int64_t ldx,
                  int64_t ldw, int64_t ldy, void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg,
                  ojx_stream_t stream);

/* Split-K partial products in fp32: parts[s][M][N] = x[:, K_s] . W[:, K_s]^T over S contiguous K ranges.
 * Replaces _skmm's torch.bmm(x.view(M,S,K/S).transpose(0,1), Wsk, out_dtype=fp32) (src/fastmodel.py:158-166)
 * and lt2_run (src/lt.cpp:160-169); W stays [N,K] (no [S,K/S,N] copy). Split s covers K range
 * [s*c, min(K,(s+1)*c)) with c = K/S rounded up to a multiple of 8, i.e. the reference's K/S chunks whenever
 * K is a multiple of 8*S. tile < 0 = the plan's tile. */
int ojx_gemm_splitk_f32(const void* x, const void* w, float* parts, int64_t M, int64_t N, int64_t K, int64_t ldx,
                        int64_t ldw, int32_t S, int32_t tile, ojx_stream_t stream);

/* out[M,I] = bf16(bf16(silu(g)) * u) with [g | u] = x . W_gu^T, W_gu packed by ojx_pack_gate_up ([2I, K]).
 * Replaces _silu_mul(_mm(hn, w_gu)) (src/fastmodel.py:478,190-194; src/kernels.cu:1304-1331) in one pass. */
int ojx_gemm_silu_mul(const void* x, const void* w_gu_packed, void* out, int64_t M, int64_t I, int64_t K,
                      void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg, ojx_stream_t stream);

/* h_out = bf16(residual + bf16(x . W^T)); if hn_out != NULL also
 * hn_out = bf16((h * rsqrt(mean(h^2) + eps)) * w1), zero on rows where rowmask == 0 (rowmask may be NULL).
 * Replaces _res (src/fastmodel.py:196-203): split-K GEMM + add_rmsnorm_sk2 (src/kernels.cu:1444-1501) or
 * GEMM + add_rmsnorm (src/kernels.cu:41-73). h_out may alias residual. RMSNorm needs N % 8 == 0, N/8 <= 1024. */
int ojx_gemm_residual_rmsnorm(const void* x, const void* w, const void* residual, const float* w1,
                              const int32_t* rowmask, float eps, void* h_out, void* hn_out, int64_t M, int64_t N,
                              int64_t K, void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg,
                              ojx_stream_t stream);

/* Load-time weight layout: W [N, K] row-major -> wp [K/64][N/16][16][64] bf16 (N % 16 == 0, K % 64 == 0, at most
 * 2 GiB). The 16-row x 64-k blocks of one 64-k stage of all rows are contiguous, so the weights a workgroup streams
 * for one stage of its tile are one contiguous run instead of one 128-byte piece per row (measured on MI355X: a
 * weight stream of 144-row tiles reads 6.8 TB/s against 6.5 row-major). For the fused gate-up, pack the output of
 * ojx_pack_gate_up. Replaces the load-time weight re-layout of _split (src/fastmodel.py:86-112, 186-188) with one
 * copy in a layout the kernels stream; the row-major W is no longer needed once packed. */
int ojx_pack_weight(const void* w, void* wp, int64_t N, int64_t K, ojx_stream_t stream);

/* The reference's split-K weight copy back to W: wsk [S, K/S, N] bf16 (wsk[s][k][n] = W[n][s K/S + k], made by _split,
 * src/fastmodel.py:186-188, and taken by lt2_run, src/lt.cpp:58-59,160-169) -> w [N, K] row-major. For callers that
 * hold only the reference's copy: the projections read W [N, K] (or its packed layout) and split K in place. N and
 * K multiples of 8, K % S == 0. */
int ojx_unsplit_weight(const void* wsk, void* w, int64_t N, int64_t K, int64_t S, ojx_stream_t stream);

/* ojx_gemm_bf16 / ojx_gemm_silu_mul / ojx_gemm_residual_rmsnorm on a packed weight: same arguments and results (x
 * row-major as before), the weight in the ojx_pack_weight layout. Tile families 0, 5 and 6 read it; cfg NULL = the
 * plan for kind | OJX_KIND_PACKED; an explicit cfg must name a tile of those families, with no tail, and split-K
 * chunks are whole 64-k stages (ceil(K / S) rounded up to a multiple of 64). */
int ojx_gemm_bf16_pk(const void* x, const void* wp, void* y, int64_t M, int64_t N, int64_t K, int64_t ldx,
                     int64_t ldy, void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg, ojx_stream_t stream);
int ojx_gemm_silu_mul_pk(const void* x, const void* w_gu_pk, void* out, int64_t M, int64_t I, int64_t K,
                         void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg, ojx_stream_t stream);
int ojx_gemm_residual_rmsnorm_pk(const void* x, const void* wp, const void* residual, const float* w1,
                                 const int32_t* rowmask, float eps, void* h_out, void* hn_out, int64_t M, int64_t N,
                                 int64_t K, void* workspace, int64_t workspace_bytes, const ojx_cfg* cfg,
                                 ojx_stream_t stream);

/* Full-attention prep, the consumer of the full-attention layers' QKV in-projection: replaces fullattn_prep2
 * (src/kernels.cu:302-360; called as K.fullattn_prep2(proj, qw1, kw1, cos, sin, 1, N, HQ, HKV, D, eps) by
 * forward_gtree, src/fastmodel.py:462). proj [N, (2 HQ + 2 HKV) D] bf16 (per q head: D q dims then D gate dims; then
 * the k heads, then the v heads). q and k heads: RMSNorm over the head (weight qw1 / kw1 fp32 [D], eps), then the
 * rotate-half RoPE on the first RD dims with cos / sin bf16 [N, RD]; outputs qt [HQ, N, D], kt [HKV, N, D],
 * vt [HKV, N, D] (v copied) and gate [N, HQ D] (copied), all bf16. D = 256; RD = 16 * a power of two, <= D. */
int ojx_fullattn_prep(const void* proj, int64_t N, int32_t HQ, int32_t HKV, int32_t D, int32_t RD, float eps,
                      const float* qw1, const float* kw1, const void* cosb, const void* sinb, void* qt, void* kt,
                      void* vt, void* gate, ojx_stream_t stream);

/* The QKV in-projection with the prep fused into its epilogue: x [M, K] . W^T with W [(2 HQ + 2 HKV) D, K]
 * (row-major, or packed by ojx_pack_weight when w_packed != 0), then ojx_fullattn_prep's arithmetic on the bf16
 * projection of each 256-row head block, written straight to qt, kt, vt and gate: the [M, (2 HQ + 2 HKV) D]
 * projection never goes to memory and the prep launch disappears. Replaces _mm(hn, d.w_in) followed by
 * fullattn_prep2 (src/fastmodel.py:412,462). D = 256, RD = 64. Results equal _mm + ojx_fullattn_prep up to the
 * order in which a head's sum of squares is added (fp32). */
int ojx_gemm_qkv_fullattn_prep(const void* x, const void* w, int32_t w_packed, const float* qw1, const float* kw1,
                               const void* cosb, const void* sinb, void* qt, void* kt, void* vt, void* gate,
                               int64_t M, int64_t K, int32_t HQ, int32_t HKV, int32_t D, int32_t RD, float eps,
                               ojx_stream_t stream);

/* Linear-attention prep on the tree layout, the consumer of the linear-attention layers' in-projection: replaces
 * linattn_prep_dedup2 (src/kernels.cu:1176-1290; called as K.linattn_prep_dedup2(proj, lay.hist, lay.rep_ptr,
 * lay.rep_pos, lay.L2, convw, A_log, dt_bias, KD, VD, HV, HK, HD, rep_qk) by forward_gtree, src/fastmodel.py:420,438).
 * proj [N, 2 KD + 2 VD + 2 HV] bf16 (q | k | v conv channels, z, b, a); hist int32 [N + 1, 4] (rows t-3 .. t of each
 * packed row's path, -1 = none; row N unused), rep_ptr int32 [N + 2] and rep_pos int32 [R] (the CSR map from packed
 * rows to path slots, group N = end padding), convw bf16 [2 KD + VD, 4], A_log and dt_bias bf16 [HV]. Outputs:
 * q, k bf16 [R, RQ KD] with RQ = HV / HK (3) when rep_qk != 0 else 1, v bf16 [R, VD], g fp32 [R, HV], beta bf16
 * [R, HV]. Depthwise causal conv (4 taps) + SiLU, L2 norm of each q / k head, beta = sigmoid(b),
 * g = -exp(A_log) softplus(a + dt_bias); each packed row computed once and written to every slot holding it; the
 * end-padding slots get zeros. HD = 128, KD = HK HD, R a multiple of L2, HV <= 256; every pointer 16-byte aligned.
 * The index arrays are used as given (as in the reference): rep_ptr non-decreasing with rep_ptr[N + 1] <= R,
 * rep_pos entries in [0, R), hist entries -1 or in [0, N). */
int ojx_linattn_prep(const void* proj, const int32_t* hist, const int32_t* rep_ptr, const int32_t* rep_pos,
                     int64_t N, int64_t R, int64_t L2, const void* convw, const void* A_log, const void* dt_bias,
                     int32_t KD, int32_t VD, int32_t HV, int32_t HK, int32_t HD, int32_t rep_qk, void* q, void* k,
                     void* v, float* g, void* beta, ojx_stream_t stream);

/* Bytes of the static device scratch behind ojx_gemm_residual_rmsnorm_noalloc (one array per GPU). */
#define OJX_NOALLOC_SCRATCH_BYTES (32LL << 20)

/* ojx_gemm_residual_rmsnorm without a workspace argument and without any allocation: no hipMalloc / hipFree and no
 * allocating library call, on any call. No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation). The kernels' scratch (split-K
 * planes, stream-K partial tiles) lives in a file-scope device array of OJX_NOALLOC_SCRATCH_BYTES per GPU, which
 * each GPU the library runs on holds until the process ends. With cfg == NULL the plan's configuration is used with
 * its split-K count (or stream-K spread) lowered until its workspace fits the scratch; an explicit cfg whose
 * workspace exceeds the scratch is rejected with OJX_ERR_WORKSPACE. Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams, or concurrent host threads) race and must be serialized by the
 * caller. Results are bit-identical to ojx_gemm_residual_rmsnorm with the same configuration. */
int ojx_gemm_residual_rmsnorm_noalloc(const void* x, const void* w, const void* residual, const float* w1,
                                      const int32_t* rowmask, float eps, void* h_out, void* hn_out, int64_t M,
                                      int64_t N, int64_t K, const ojx_cfg* cfg, ojx_stream_t stream);

/* Scoring head: scores[r] = sum_j float(hn[lastidx[r]][j]) * w[j] + bias[0] (bias may be NULL), fp32.
 * hn bf16 [rows, H] contiguous, lastidx int64 [R], w fp32 [H], scores fp32 [R]. Replaces the last matmul of the
 * forward, mdl.head(hn[lastidx].float()).squeeze(-1) (src/server.py:37,57,129; hn[lastidx] is
 * src/fastmodel.py:314,482), with the row gather fused in. An index outside [0, rows) gives NaN for that score
 * (the reference's indexing would raise; a kernel cannot). H % 8 == 0. */
int ojx_head_scores(const void* hn, int64_t rows, int64_t H, const int64_t* lastidx, int64_t R, const float* w,
                    const float* bias, float* scores, ojx_stream_t stream);

/* Standalone epilogues, same arguments and semantics as the reference extension's functions. */
/* add_rmsnorm (src/kernels.cu:41-73, 755-767): delta may be NULL (then h_out is not written: h == x). */
int ojx_add_rmsnorm(const void* x, const void* delta, const float* w1, const int32_t* rowmask, float eps,
                    void* h_out, void* hn_out, int64_t M, int64_t H, ojx_stream_t stream);
/* add_rmsnorm_sk / add_rmsnorm_sk2 (src/kernels.cu:475-515, 1444-1501): parts fp32 [S, M, H]. */
int ojx_add_rmsnorm_sk(const void* x, const float* parts, int32_t S, const float* w1, const int32_t* rowmask,
                       float eps, void* h_out, void* hn_out, int64_t M, int64_t H, ojx_stream_t stream);
/* silu_mul (src/kernels.cu:76-89, 769-777): gu [M, 2I] = [gate | up] -> out [M, I]. */
int ojx_silu_mul(const void* gu, void* out, int64_t M, int64_t I, ojx_stream_t stream);
/* silu_mul_lut (src/kernels.cu:1304-1331): tab = the 65536-entry bf16 silu table from ojx_act_tables. */
int ojx_silu_mul_lut(const void* gu, const void* tab, void* out, int64_t M, int64_t I, ojx_stream_t stream);
/* act_tables (src/kernels.cu:1288-1301): silu_b bf16[65536], sig_f fp32[65536]. */
int ojx_act_tables(void* silu_b, float* sig_f, ojx_stream_t stream);

/* Weight layout for the fused gate-up: packed[2I, K], rows in blocks of 8 = gate rows 4b..4b+3, up rows 4b..4b+3.
 * Replaces the load-time torch.cat([gate, up]) of src/fastmodel.py:90. I must be a multiple of 4, K of 8. */
int ojx_pack_gate_up(const void* gate, const void* up, void* packed, int64_t I, int64_t K, ojx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* OJX_H */
