// kernels.h — argument blocks and launch functions of the gfx950 kernels.
// Every launch function checks the shapes its kernel assumes and returns a TSN_* status; the
// kernels themselves carry no bounds checks beyond the tails they are written for.
#pragma once
#include "tsn_common.h"

namespace tsn {

/* ------------------------------------------------------------------ GEMM (MFMA) */
// C[M,N] = A[M,K] · W[N,K]ᵀ with f16 operands and f32 accumulation; 128x128x64 tiles,
// v_mfma_f32_16x16x32_f16 (pipelined kernel: 8 waves, 5 direct-to-LDS stages).
enum GemmEpi { EPI_STORE = 0, EPI_RESID = 1, EPI_QKV = 2, EPI_SWIGLU = 3, EPI_SNAKE = 4, EPI_RSNAKE = 5 };

struct GemmProblem {
    // A operand rows (f16, or f32 converted on load): row m -> rowmap_phys(amap, m).
    const void *A; int lda; RowMap amap;
    // Convolution view of K: K = taps*Kc; column k reads channel k % Kc of source row
    // t - pad + (k / Kc)*dil of the same sample, zero outside [0, a_T). taps = 1, pad = 0 is a GEMM.
    // dil > 1 (dilated taps) only with EPI_SNAKE.
    int taps, Kc, pad, a_T, dil;
    const half_t *W; int ldw;          // [N][K] row-major
    // w_half: the A operand is an f16 hi|lo pair per tap (Kc = 2*IC: hi channels, then lo) and W
    // holds IC channels per tap ([N][taps][IC], ldw >= taps*IC); both halves read the same W columns
    int w_half;
    const float *bias;                 // [N] or null
    int M, N, K;
    // EPI_STORE: Y[ymap(m)*ldy + n] = act(acc + bias), f16 or f32
    // EPI_SWIGLU: W rows interleaved in 64-row blocks (w1 block j, then w3 block j), N = 2F;
    // Y[ymap(m)*ldy + 64j + c] = silu(w1 row 64j+c · a) * (w3 row 64j+c · a), f16, no bias
    void *Y; int ldy; RowMap ymap; int y_f16; int silu;
    // f16 Y (EPI_STORE, EPI_SWIGLU): nonzero also writes lo = f16(y - f16(y)) at column offset y_lo
    // of the same row (hi|lo operand of a following GEMM against [W | W]); K is then never split
    int y_lo;
    // EPI_SNAKE: y = snake(acc + bias) = v + sin(v*ea[n])^2 * eb[n] with snake = [ea (N) | eb (N)],
    // stored f16 as a three-part row: hi at column n, lo = f16(y - hi) at n + y_lo, hi again at
    // n + y_hi2 ([hi | lo | hi], the operand of a following GEMM against [W_hi | W_hi | W_lo]);
    // K is never split
    int y_hi2;
    const float *snake;
    // EPI_RSNAKE: x = (r_add ? R[rmap(m)*ldr + n] : 0) + acc + bias[n] is stored to R, and snake(x) (table
    // as EPI_SNAKE) as a three-part f16 row: columns come in phases of C = y_lo, and column n of phase
    // n / C lands at n + 2C*(n / C) (hi), + C (lo), + 2C (hi) of Y row ymap(m)*ldy
    int r_add;
    // EPI_RESID: R[rmap(m)*ldr + n] += gate[(m / gate_L)*gate_ld + n] * (acc + bias)
    float *R; int ldr; RowMap rmap; const float *gate; int gate_ld; int gate_L;
    // EPI_QKV: columns [0,Hq) q, [Hq,2Hq) k, [2Hq,3Hq) v; heads of hd = 64 columns.
    // Row m -> sample b = m / q_L, position s = q_soff + m % q_L.
    // q, k: per-head RMSNorm (weights qn/kn), RoPE for (m % q_L) < rope_len, q *= q_scale;
    // stored to Q/Kd [b][h][S_att][64]; v stored transposed to Vt [b][h][64][Sp].
    half_t *Q, *Kd, *Vt; int S_att, Sp, nh, Hq, q_L, q_soff, rope_len;
    const float *qn, *kn; float rms_eps, q_scale;
    const float *rope;                 // [pos][32][2] (cos, sin)
    // filled by the launcher
    int tile_start, tiles_m, tiles_n;
    long long unit_start;              // stream-K: first (tile, K tile) unit of this problem
    // split-K (filled by the launcher): splits > 1 writes f32 partials [splits][M][N] at ws, and a
    // second kernel sums them in split order and applies the epilogue
    int splits;
    float *ws;
};

// Weight lines a kernel touches for a GEMM that runs after it, so that GEMM's reads of them come
// from the last-level cache instead of HBM: the first row_bytes of each of `rows` rows, ld bytes
// apart (row_bytes and ld multiples of 128; inside one allocation). Extra workgroups of the
// launch (prefetch.h) load one dword per 128-byte line and do nothing else, so the launch's other
// workgroups never wait for them: at the front of an LN grid (dispatched first), after the tiles
// of a data-parallel GEMM grid (on the CUs its last round leaves free). rows = 0: nothing.
struct PfRange {
    const void *p = nullptr;
    int rows = 0, row_bytes = 0;
    long long ld = 0;
};
constexpr int PF_PER_LANE = 2;   // loads per lane of a prefetch workgroup
constexpr int PF_RANGES = 4;     // ranges per launch
// prefetch workgroups of `waves` waves that cover every range; false if a range is malformed
bool pf_ranges_ok(const PfRange (&pf)[PF_RANGES]);
int pf_workgroups(const PfRange (&pf)[PF_RANGES], int waves);

/* ------------------------------------------------------------------ GEMV */
// Y[b*ldy + n] = sum_k W[n*ldw + k] X[b*ldx + k] (+ bias[n], + addv[b*ld_add + n], SiLU) for the
// nb rows b of X; Y2 (optional) = silu of the value written to Y.
struct GemvArgs {
    const void *W; int ldw; int wdt;
    const float *X; int ldx;
    float *Y; int ldy;
    const float *bias;
    const float *addv; int ld_add;
    float *Y2; int ldy2;
    int N, K, nb, silu;
};

struct GemmBatch {
    GemmProblem p[3];
    int nprob = 0;
    int total_tiles = 0;
    // optional f32 workspace for split-K partials (EPI_RESID / EPI_STORE) and stream-K partial
    // tiles (any epilogue); null disables both
    float *ws = nullptr;
    size_t ws_bytes = 0;
    // set by gemm_plan: pipelined kernel chosen, and the symbol of the kernel that will run
    int pipe = 0;
    const char *kname = nullptr;
    // stream-K schedule (gemm_plan, pipelined kernel with a workspace): sk_g workgroups share the
    // sk_units (tile, K tile) units evenly; partial tiles go to ws. With sk_cnt (zero-initialised
    // arrival counters, sk_cnt_n >= total tiles; every launch leaves them at zero) the last
    // contributor of a cut tile finishes it inside the kernel; otherwise launch_gemm_reduce does
    // (gemm_fixup_kernel)
    int sk = 0, sk_g = 0;
    long long sk_units = 0;
    unsigned *sk_cnt = nullptr;
    int sk_cnt_n = 0;
    int hl = 0;   // some problem reads half-width W (selects the kernel variant)
    // nonzero: never stream-K, and choose the classic K split by the estimated time (waves x K tiles
    // per split, plus the partial-sum traffic). For long-K GEMMs with few tiles, whose A and W tiles
    // would not be shared in L2 under stream-K's staggered K ranges.
    int split_waves = 0;
    // the split_waves estimate's fixed cost of a split (the reduce), in K-tile times: about 2 for
    // launches replayed from a captured graph; an eager launch from the host costs about 10
    float split_overhead = 2.0f;
    // nonzero (EPI_RESID or EPI_STORE, pipelined-kernel operands, no half-width W, no hi|lo
    // output): 64x64 tiles over the full K (gemm_small_kernel), no split and no stream-K, for
    // one-tap problems when the 128x128 grid has fewer than 256 tiles. gemm_plan clears it
    // otherwise (and for a plain store whose operands the kernel does not take, where a residual
    // request is an error), and the workspace then serves the usual split-K / stream-K choice; it
    // sets 2 for the two-group kernel (gemm_small2_kernel) when the grid holds at most one
    // workgroup per CU.
    int small = 0;
    // set by gemm_plan: the two-stage kernel (gemm_pipe2_kernel, two workgroups per CU) for
    // data-parallel grids of more than one round (256 tiles)
    int ns2 = 0;
    // set by gemm_plan: 256x256 tiles (gemm_wide_kernel) for data-parallel grids of several rounds
    // whose 256x256 grid still fills the chip; tiles_m/tiles_n/tile_start then count 256x256 tiles
    int wide = 0;
    // nonzero: A and W hold bf16 values and the MFMAs run bf16 products (gemm_pipe_bf16_kernel /
    // gemm_pipe2_bf16_kernel: EPI_STORE with f32 Y, one tap, data-parallel, no split)
    int bf16 = 0;
    // weights of a following GEMM to touch from extra workgroups launched after the tiles (they
    // take the CUs the last round leaves free); data-parallel pipelined kernels only, else ignored.
    // pf_nwg is set by gemm_plan.
    PfRange pf[PF_RANGES];
    int pf_nwg = 0;
    // rows of an HBM-bound GEMV (gv.N > 0; BF16 W, two rows of X, K = 1024) for extra workgroups
    // launched after the tiles, on the CUs a single-round data-parallel pipelined grid leaves free;
    // each then runs its share of the prefetch chunks (no prefetch workgroups of their own).
    // gemm_plan sets gv_nwg; where it stays 0 the launcher runs the GEMV as its own kernel just
    // before the GEMM.
    GemvArgs gv{};
    int gv_nwg = 0;
};

// a_f32: A operand is f32 (converted to f16 on load). All problems share the epilogue kind.
// With a workspace (EPI_RESID / EPI_STORE, pipelined kernel) the launcher may split K; the
// partial sums are then reduced and the epilogue applied by launch_gemm_reduce, which must follow
// on the same stream (it returns at once when no problem was split).
int launch_gemm(GemmBatch &b, int epi, bool a_f32, hipStream_t st);
// launch_gemm = gemm_plan (checks, tiling, split-K choice, kernel choice) + gemm_launch_planned
int gemm_plan(GemmBatch &b, int epi, bool a_f32);
int gemm_launch_planned(const GemmBatch &b, int epi, bool a_f32, hipStream_t st);
int launch_gemm_reduce(const GemmBatch &b, int epi, hipStream_t st);
bool gemm_needs_reduce(const GemmBatch &b);
// symbol of the kernel launch_gemm_reduce runs for this batch
const char *gemm_reduce_name(const GemmBatch &b, int epi);
void gemm_problem_init(GemmProblem &p);

/* ------------------------------------------------------------------ attention */
// Flash attention, hd = 64, non-causal, no mask. Q/K [BH][S][64] f16, Vt [BH][64][Sp] f16
// (keys >= S of Vt must hold finite values; the library keeps them zero). Q holds q * softmax
// scale * log2(e): its producer folds the factor in before the f16 rounding (the QKV epilogue's
// q_scale, launch_attn_pack's q_scale), so a product q.k is the score in log2 units.
// O row for (b, s) is rowmap_phys(omap, b*S + s); head h writes columns h*64..h*64+63.
struct AttnArgs {
    const half_t *Q, *K, *Vt;
    int S, Sp, nh, BH;
    void *O; int o_f32; int ldo; RowMap omap;
    int o_lo;           // f16 O: nonzero also writes lo = f16(o - f16(o)) at column offset o_lo
};
int launch_attention(const AttnArgs &a, hipStream_t st);

// Pack f32 q/k/v column slices of a [S, ld] buffer into Q/K [nh][S][64] and Vt [nh][64][Sp]
// (f16; Q = f16(q * q_scale); Vt keys in [S, Sp) zeroed).
int launch_attn_pack(const float *qkv, float q_scale, int S, int nh, int ld, int q_off, int k_off, int v_off,
                     half_t *Q, half_t *K, half_t *Vt, int Sp, hipStream_t st);

/* ------------------------------------------------------------------ LayerNorm + adaLN modulate */
// y = LN(x; eps, no affine) * (1 + scale) + shift, one wave per row, H % 256 == 0, H <= 2048.
// Virtual row v of segment s: x row xmap(v), y row ymap(v), sample b = v / mod_L,
// shift = mod[b*mod_ld + shift_off + c], scale = mod[b*mod_ld + scale_off + c].
struct LnSeg {
    const float *X; int ldx; RowMap xmap;
    void *Y; int ldy; RowMap ymap;
    const float *mod; int mod_ld, mod_L, shift_off, scale_off;
    int rows;
};
struct LnArgs {
    LnSeg seg[3];
    int nseg, H;
    float eps;
    PfRange pf[PF_RANGES];
    int pf_nwg;   // set by the launcher: prefetch workgroups, ahead of the row workgroups
};
// ymode: 0 f32 output, 1 f16 output, 2 f16 hi|lo pair (y_hi at column c, y_lo = f16(y - y_hi) at
// column H + c; ldy >= 2H): an f16 GEMM over [hi|lo] against a [W|W] weight reproduces the f32 y.
enum { LN_F32 = 0, LN_F16 = 1, LN_F16_HILO = 2 };
int launch_ln_mod(const LnArgs &a, int ymode, hipStream_t st);

/* ------------------------------------------------------------------ split-K reduce + residual + LN */
// One wave per row of H columns (H % 256 == 0), for the rows of up to two GEMM problems:
//   if splits > 1: x = X[row] + gate[b] * (sum_ks ws[ks][m] + bias), stored back to X
//   (splits <= 1: the GEMM epilogue already updated X; x = X[row]);
//   then, when ln is set and (m % mod_L) < ln_len: y = LN(x)*(1 + scale) + shift -> Y (f16, or f16
//   hi|lo pair), shift/scale = mod[(m / mod_L)*mod_ld + shift_off / scale_off + c].
struct RedLnSeg {
    const float *ws; int splits, M;
    const float *bias; const float *gate; int gate_ld, gate_L;
    float *X; int ldx; RowMap xmap;
    int ln, ln_len;
    const float *mod; int mod_ld, mod_L, shift_off, scale_off;
    void *Y; int ldy; RowMap ymap;
    int hilo;   // this segment's LN output as an f16 hi|lo pair (lo at column H + c) whatever ymode
};
struct RedLnArgs {
    RedLnSeg seg[3];
    int nseg, H, ymode;
    float eps;
    PfRange pf[PF_RANGES];
    int pf_nwg;   // set by the launcher: prefetch workgroups, ahead of the row workgroups
};
int launch_reduce_ln(const RedLnArgs &a, hipStream_t st);

/* ------------------------------------------------------------------ calibration probes */
// nwg workgroups x 8 waves, each wave 16 x iters MFMAs 16x16x32 f16 (16384 flops each); out holds
// nwg*512 floats
int launch_mfma_peak(float *out, int nwg, int iters, hipStream_t st);
// dst[i] = src[i] for n4 float4 elements
int launch_copy_peak(const float *src, float *dst, size_t n4, hipStream_t st);

/* ------------------------------------------------------------------ GEMV (small M) */
// Y[b][n] = act(sum_k W[n][k] * X[b][k] + bias[n] + addv[b][n]); optional Y2 = silu(Y).
// W is bf16, f16 or f32 (wdt); X, Y f32; nb <= 16 rows of X. HBM-bound: one wave per 4 rows of W
// on the VALU, or, for 16 rows of X with bf16 W and K = 256, 512 or 1024, 16 rows of W per wave on
// MFMA with X split exactly into three bf16 terms.
int launch_gemv(const GemvArgs &a, hipStream_t st);

/* ------------------------------------------------------------------ f32 SIMT linear */
// Y[ymap(m)*ldy + n] = sum_k X[xmap(m)*ldx + k] * W[n*ldw + k] + bias[n]; W bf16 / f16 / f32.
// Used where an f32 operand matters more than MFMA rate (K <= 1024 projections, f32 weights).
struct LinArgs {
    const float *X; int ldx; RowMap xmap;
    const void *W; int ldw; int wdt;
    const float *bias;
    float *Y; int ldy; RowMap ymap;
    int M, N, K;
};
int launch_linear_f32(const LinArgs &a, hipStream_t st);

/* ------------------------------------------------------------------ final layer */
// v[r] = (LN(x_r; eps)*(1 + scale) + shift) . W^T + bias for the audio rows r < rows (x row
// xmap(r), sample r / mod_L), W f16 [N][ldw] (first H columns), N <= 64 and a multiple of 16,
// H a multiple of 256 up to 2048; f32 statistics, f32-accurate product (hi|lo operand).
struct FinalArgs {
    const float *X; int ldx; RowMap xmap;
    const float *mod; int mod_ld, mod_L, shift_off, scale_off;
    const half_t *W; int ldw;
    const float *bias;
    float *Y; int ldy;
    int rows, H, N;
    float eps;
};
int launch_final_out(const FinalArgs &a, hipStream_t st);

/* ------------------------------------------------------------------ small kernels */
int launch_temb_sinusoid(const float *t, float *out, int nb, int D, float max_period, hipStream_t st);
// dst[dmap(m)*ldd + c] = src[smap(m)*lds + c], c < H (f32)
int launch_copy_rows(const float *src, int lds, RowMap smap, float *dst, int ldd, RowMap dmap,
                     int M, int H, hipStream_t st);
// sampler step on x2 [2P][n]: v = vu + (vc - vu)*cfg; x += dt*v; both arms of prompt p get x.
int launch_cfg_euler_pairs(const float *V, float *x2, int P, int n, float cfg, float dt, hipStream_t st);
// x f32 rows -> out [M][2K] f16: out[m][k] = hi = f16(x), out[m][K + k] = f16(x - hi)
int launch_split_hilo(const float *x, int ldx, RowMap xmap, half_t *out, int M, int K, hipStream_t st);
// one launch at the start of an evaluation: temb = sinusoid(t) (skipped when t is null), z2 =
// hi|lo split of z, and cM rows copied csrc -> cdst (each part as its standalone kernel)
struct EvalPrepArgs {
    const float *t; float *temb; int tnb, tD; float tmax;
    const float *z; int ldz; RowMap zmap; half_t *z2; int sM, sK;
    const float *csrc; int clds; RowMap csmap; float *cdst; int cldd; RowMap cdmap; int cM, cH;
};
int launch_eval_prep(const EvalPrepArgs &a, hipStream_t st);
// bf16 [N][K] -> f16 [N][2K] = [W | W] (weight of a GEMM over a hi|lo operand)
int launch_dup_cols_bf16_to_f16(const uint16_t *src, half_t *dst, int N, int K, hipStream_t st);
// format conversions
int launch_bf16_to_f16(const uint16_t *src, half_t *dst, size_t n, hipStream_t st);
int launch_bf16_to_f32(const uint16_t *src, float *dst, size_t n, hipStream_t st);
int launch_f16_to_f32(const half_t *src, float *dst, size_t n, hipStream_t st);
// conv weight [OC][IC][K] (bf16 or f16, src_bf16 selects) -> [OC][K][IC] f16
int launch_conv_weight_reorder(const void *src, int src_bf16, half_t *dst, int OC, int IC, int K, hipStream_t st);

// Upload-time weight layout (source [OC][IC][KT] stored as src_type, KT = 1 for a linear weight or a
// vector): destination row r(oc) = (oc % ra)*rb + (oc / ra)*rc + rd (ra = 1, rb = 0, rc = 1, rd = 0
// keeps the order), tap-major [KT][IC] within the row, channels written twice ([w | w]) when dup;
// f16 with the reference upload's f32 -> f16 rounding, or f32 when out_f32. Every r(oc) must lie in
// [0, dst_rows). Source types are the GGUF encodings the reference's loader takes
// (src/gguf.cpp to_f32): BF16 exact, F32, F16 with subnormals flushed to zero, and Q8_0 (blocks of
// 32 elements: f16 scale, 32 int8; value = scale * q), so a checkpoint's raw tensor bytes can be
// converted on the device.
enum { WP_SRC_BF16 = 0, WP_SRC_F32 = 1, WP_SRC_F16 = 2, WP_SRC_Q8_0 = 3 };
int launch_weight_prep(const void *src, int src_type, void *dst, int out_f32, int OC, int IC, int KT, int dup, int ra,
                       int rb, int rc, int rd, long long dst_rows, hipStream_t st);
// y = silu(x[m] + v[m / L]) (x [M][H], v [M/L][H] f32) as f16 hi|lo rows [M][2H] (LN_F16_HILO layout)
int launch_bcast_add_silu_f16(const float *x, const float *v, half_t *y, int L, int M, int H, hipStream_t st);

// out [M][2K] f16 hi|lo of x[m][k] + pe[m % P][k] (pe null: x alone)
int launch_add_period_hilo(const float *x, const float *pe, int P, half_t *out, int M, int K, hipStream_t st);
// VAE decoder (vae.hip). split3: f32 rows [rows][C] (C % 8 == 0) -> f16 [rows][3C], v = x or, with a
// table ab = [exp(alpha) (C) | exp(-beta) (C)], snake(x) = x + sin(x*ea)^2*eb; parts [hi | lo | hi]
// (lo_part 1, activation operand) or [hi | hi | lo] (lo_part 2, weight operand)
int launch_split3(const float *x, long long rows, int C, const float *ab, int lo_part, half_t *out, hipStream_t st);
// y [T][OC] = conv(snake(x), W [OC][C][KK], pad), no bias; x [T][C] f32, OC in {1, 2, 4}, KK == 7, C % 8 == 0
int launch_conv_out(const float *x, const float *ab, const float *W, float *y, int T, int C, int OC, int KK, int pad,
                    hipStream_t st);
// Text encoders (enc.hip), all f32.
// gemm_f32: Y[m*ldy + n] = act(sum_k A[m*lda + k] W[n*ldw + k] + bias[n]) (act 1: quick GELU), or with
// resid set Y[m*ldy + n] += sum + bias[n]; K % 4 == 0, f32 MFMA. With a workspace the launcher may
// split K (partials reduced in split order by a second kernel it launches); splits and kps are its own.
struct EncGemmArgs {
    const float *A; int lda;
    const float *W; int ldw;
    const float *bias;
    float *Y; int ldy;
    int M, N, K;
    int resid, act;
    float *ws; size_t ws_bytes;
    int splits, kps;
};
int launch_gemm_f32(const EncGemmArgs &g, hipStream_t st);
// LayerNorm with weight and bias (ln) or RMSNorm with weight, rows of H floats
int launch_enc_norm(const float *x, float *y, const float *w, const float *b, int rows, int H, float eps, bool ln,
                    hipStream_t st);
// attention over one context of S <= 128 rows, heads of 64: q, k, v at column offsets q_off/k_off/v_off
// + 64h of qkv rows (stride ld), output at column 64h of out rows (stride ldo);
// mode 0 none, 1 T5 (keys with pad[k] == 0 masked, else + rel[bucket[q*S + k]*nh + h]),
// 2 CLIP (keys k > q or k > eot masked)
struct EncAttnArgs {
    const float *qkv; int ld, q_off, k_off, v_off;
    float *out; int ldo;
    int S, nh, hd;
    float scale;
    int mode;
    const int32_t *bucket; const float *rel; const int32_t *pad;
    int eot;
};
int launch_enc_attention(const EncAttnArgs &a, hipStream_t st);
// y[r][c] = gelu_tanh(u[r][c]) * u[r][F + c], u rows of 2F
int launch_geglu_rows(const float *u, float *y, int rows, int F, hipStream_t st);
// x[s][:] = tok[ids[s]][:] (+ pos[s][:]); ids on the device, each inside tok's rows
int launch_embed_rows(const int32_t *ids, const float *tok, const float *pos, float *x, int S, int H, hipStream_t st);
// dst[i][:] = src[idx[i]][:] for rows x H floats (idx on the device, every entry a valid src row)
int launch_gather_rows(const float *src, const int32_t *idx, float *dst, int rows, int H, hipStream_t st);
// out[c] = mean over rows of x[r][c], rows summed in order (src/net.mm Runtime::mean_cols)
int launch_mean_rows(const float *x, int rows, int H, float *out, hipStream_t st);

/* ------------------------------------------------------------------ net.h conv surface (netops.hip) */
// Geometry of Runtime::conv (src/net.h:29-34): x [T][IC] rows of stride ldx -> y [OL][OC].
struct ConvGeom {
    int T, OL, IC, OC, K, stride, pad, dil, convt, ldx;
};
// Columns of a prepared conv weight row: K*IC (f16/bf16 source) or 3*K*IC (f32 source, three
// parts per tap) rounded up to a multiple of 64.
int conv_prep_cols(int sdt, int IC, int K);
// W [OC][IC][K] (sdt f16, bf16 or f32) -> Wp [OC][conv_prep_cols] f16, tap-major, zero padded:
// f16/bf16 sources one channel per column (bf16 with the reference upload's rounding), f32
// sources [hi | hi | lo] of each tap's channels (the weight of a three-part product)
int launch_conv_prepare(const void *W, int sdt, half_t *Wp, int OC, int IC, int K, hipStream_t st);
// gathered operand rows [t0, t0 + rows) of the conv (the reference's im2col, src/net.mm:36-48):
// parts 1 -> [rows][2*Kp] f16 hi|lo halves; parts 3 -> [rows][Kp] with [hi | lo | hi] per tap
int launch_conv_gather(const float *x, const ConvGeom &g, int t0, int rows, int parts, int Kp, half_t *out,
                       hipStream_t st);
// direct f32 conv on a prepared weight (outputs too narrow for a GEMM tile)
int launch_conv_direct(const float *x, const ConvGeom &g, const half_t *Wp, int parts, int Kp, const float *bias,
                       float *y, hipStream_t st);
// LayerNorm without affine, rows of H floats (shaders/ops_conv.metal:77-89)
int launch_ln_plain(const float *x, float *y, int S, int H, float eps, hipStream_t st);
// y = gelu_tanh(a) * b (shaders/ops_conv.metal:15-24); x = gelu_quick(x) (:25-29)
int launch_geglu(const float *a, const float *b, float *y, size_t n, hipStream_t st);
int launch_gelu_quick(float *x, size_t n, hipStream_t st);
// element-interleaved qkv rows [rows][3H] -> block q|k|v rows [row_off + r][3H] (shaders/ops_conv.metal:60-74)
int launch_qkv_split3(const float *src, float *dst, int rows, int H, int row_off, hipStream_t st);

// reference-surface elementwise ops (f32)
int launch_silu(float *x, size_t n, hipStream_t st);
int launch_copy(const float *x, float *y, size_t n, hipStream_t st);
int launch_swiglu(const float *a, const float *b, float *y, size_t n, hipStream_t st);
int launch_add(const float *a, const float *b, float *y, size_t n, hipStream_t st);
int launch_add_bcast_col(const float *x, const float *v, float *y, int S, int H, hipStream_t st);
int launch_cfg_euler(const float *fc, const float *fu, float *x, size_t n, float cfg, float dt, hipStream_t st);
int launch_gate_add(const float *x, const float *f, const float *mod, float *y, int rows, int H,
                    int per_row, int chunks, int gate_idx, hipStream_t st);
int launch_rms_head(float *x, const float *w, int rows, int nh, int ld, int hd, int col_off, int row_off,
                    float eps, hipStream_t st);
int launch_rope_pairs(float *x, const int32_t *pos, int rows, int nh, int ld, int hd, int col_off,
                      int row_off, float fscale, float base, hipStream_t st);

} // namespace tsn
