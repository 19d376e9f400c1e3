/* tsn.h — C ABI of the MI355X (gfx950) DiT velocity path: libtsn.so.
 *
 * Drop-in boundary for the ThinkSound-native hot path. Each entry point names the reference
 * interface it replaces (path:line into the ThinkSound-native sources). All pointers to tensors are
 * DEVICE pointers obtained from tsn_alloc unless the parameter name ends in _host. Every call
 * returns a tsn_status (0 = ok); on failure tsn_last_error() returns a message for the calling
 * thread. Launchers are asynchronous on the runtime's single HIP stream (the reference batches
 * into one Metal command buffer, src/gpu.mm:118-162); tsn_commit / tsn_sync wait.
 * A runtime handle is not re-entrant: calls on one handle must not overlap.
 *
 * Layout conventions: row-major; GEMM weights [N][K] (out, in); conv weights [OC][IC][K] in the
 * reference's layout, prepared once with tsn_conv1d_prepare.
 */
#ifndef TSN_H
#define TSN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    TSN_OK = 0,
    TSN_ERR_ARG = 1,          /* invalid argument (null pointer, bad shape) */
    TSN_ERR_HIP = 2,          /* HIP runtime error */
    TSN_ERR_UNSUPPORTED = 3,  /* valid but not implemented on this path (e.g. strided conv) */
    TSN_ERR_OOM = 4,          /* device allocation failed */
    TSN_ERR_STATE = 5         /* call out of order */
} tsn_status;

typedef enum { TSN_F32 = 0, TSN_F16 = 1, TSN_BF16 = 2 } tsn_dtype;

typedef struct tsn_runtime tsn_runtime;
typedef struct tsn_dit tsn_dit;

const char *tsn_last_error(void);
int tsn_version(void);

/* ---------------- device harness: replaces tn::gpu::Device (src/gpu.h:20-48) ---------------- */
int tsn_runtime_create(int device, tsn_runtime **out);          /* Device::init   src/gpu.h:25 */
int tsn_runtime_destroy(tsn_runtime *rt);                       /* Device::~Device src/gpu.h:22 */
int tsn_alloc(tsn_runtime *rt, size_t bytes, void **dptr);      /* Device::alloc  src/gpu.h:26; zero-filled */
int tsn_free(tsn_runtime *rt, void *dptr);                      /* (no reference counterpart: Metal buffers live
                                                                    for the process, src/gpu.mm:52-64) */
/* Unified memory is replaced by explicit copies (host writes to Buf.p: src/dit_fwd.cpp:120-121,
 * src/pipeline.cpp:131-132). Both block until the copy is done. */
int tsn_upload(tsn_runtime *rt, void *dptr, const void *src_host, size_t bytes);
int tsn_download(tsn_runtime *rt, void *dst_host, const void *dptr, size_t bytes);
int tsn_begin(tsn_runtime *rt);                                 /* Device::begin  src/gpu.h:31 */
int tsn_commit(tsn_runtime *rt);                                /* Device::commit src/gpu.h:38 */
double tsn_last_gpu_ms(tsn_runtime *rt);                        /* Device::last_gpu_ms src/gpu.h:40 */
int tsn_sync(tsn_runtime *rt);
/* Live device allocations this runtime owns: their number and bytes (as requested). No reference
 * counterpart (Metal buffers are never freed); lets a caller check that a call allocated nothing. */
int tsn_runtime_alloc_stats(tsn_runtime *rt, size_t *count, size_t *bytes);

/* ---------------- launcher runtime: tn::Runtime (src/net.h:18-51) ---------------- */
/* Y[M,N] = X[M,K]·W[N,K]^T (+bias[N], f32). Runtime::gemm src/net.h:24-26, src/net.mm:14-23.
 * wdtype TSN_F16 with f32 X keeps the reference's f32-activation contract (gemm_mpp_h,
 * shaders/gemm_mpp.metal:19-25): X is split into an f16 hi|lo pair on the device and multiplied
 * against [W | W] on MFMA with f32 accumulation, so the product is f32-accurate (relative error
 * about 2^-22 of the operand, against 2^-11 for an f16-rounded X). Y f32, or f16 on request. Shapes
 * the MFMA tiling does not take (K % 64, N % 8, unaligned W/bias/Y) run exact f32 products on the
 * SIMT path (f32 Y only). wdtype TSN_F16 with f16 X is the plain f16 product (opt-in, f16 operands
 * as given). TSN_F32 / TSN_BF16 weights run the f32 SIMT path (X, Y f32). TSN_BF16 weights with
 * TSN_BF16 X run bf16 products on MFMA (f32 accumulation, f32 Y; K % 64 == 0, N % 8 == 0, 16-byte
 * aligned rows, else TSN_ERR_UNSUPPORTED): the bf16-operand mode, beside the f16 one. ld* = 0 means packed.
 * Uses the runtime's grow-on-demand scratch (2*M*K halves). On the f16-W MFMA routes a long K over
 * few 128x128 output tiles is split: the parts' f32 partial sums go to the runtime's fixed 32 MiB
 * workspace (allocated by tsn_runtime_create) and are summed in split order, so results stay
 * deterministic. */
int tsn_gemm(tsn_runtime *rt, int wdtype, const void *W, const void *X, int xdtype, void *Y, int ydtype,
             const float *bias, uint32_t M, uint32_t N, uint32_t K, uint32_t ldx, uint32_t ldw, uint32_t ldy);
/* tsn_gemm without any device allocation. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments, kernels and results as tsn_gemm (bit-identical; a K split uses
 * the workspace tsn_runtime_create allocated); the f16 hi|lo
 * split of an f32 X goes to a fixed 32 MiB device array per GPU instead of the runtime's scratch, so
 * with f16 W and f32 X it needs M*K <= tsn_gemm_noalloc_max_elems() (TSN_ERR_ARG beyond). The array
 * is shared by every call on one GPU and keeps the last call's contents (nothing in it needs to
 * start at zero). Calls on one GPU are ordered on the device: a call from another stream (another
 * runtime) waits for the previous call's GEMM through a per-GPU event. Calls made while the stream
 * is being captured into a graph are not ordered that way: the caller orders the graph's launches
 * against other users of the array. */
int tsn_gemm_noalloc(tsn_runtime *rt, int wdtype, const void *W, const void *X, int xdtype, void *Y, int ydtype,
                     const float *bias, uint32_t M, uint32_t N, uint32_t K, uint32_t ldx, uint32_t ldw, uint32_t ldy);
size_t tsn_gemm_noalloc_max_elems(void);
/* y[n] = bias[n] + W[n,:]·x. Runtime::gemv src/net.h:27-28, src/net.mm:51-56 (wdtype f16/bf16/f32). */
int tsn_gemv(tsn_runtime *rt, const void *W, int wdtype, const float *x, float *y, const float *bias,
             uint32_t N, uint32_t K, uint32_t ldw);
/* Upload-time conv weight transform, W [OC][IC][K] in the reference's layout (wdtype TSN_F16, TSN_BF16
 * or TSN_F32; the reference converts at load, src/net.mm:141-168) -> Wp, tap-major f16 rows that
 * tsn_conv1d reads as an implicit GEMM: f16/bf16 weights one f16 per element (bf16 with the
 * reference upload's rounding), f32 weights [hi | hi | lo] f16 parts per tap (f32-accurate
 * products). Wp must hold tsn_conv1d_prepared_bytes(wdtype, OC, IC, K) bytes. */
size_t tsn_conv1d_prepared_bytes(int wdtype, uint32_t OC, uint32_t IC, uint32_t K);
int tsn_conv1d_prepare(tsn_runtime *rt, const void *W, int wdtype, void *Wp, uint32_t OC, uint32_t IC, uint32_t K);
/* conv1d, x [T,IC] f32, y [OL,OC] f32 (+bias). Runtime::conv src/net.h:29-34, src/net.mm:25-49, with
 * the im2col semantics of shaders/ops_conv.metal:226-236,266-283: tap k of output row t reads row
 * t*stride - pad + k*dil, or, when convt, row (t - pad + k)/stride of the zero-stuffed input where
 * t - pad + k is a non-negative multiple of stride; zero outside [0, T). Wp is the output of
 * tsn_conv1d_prepare for the same wdtype (wf16 true: TSN_F16/TSN_BF16; false: TSN_F32). f32-accurate
 * for every weight dtype. Stride 1, dilation 1 and IC % 64 == 0 run as an implicit GEMM (taps in K);
 * other geometries gather the operand in chunks of at most 64 MB of scratch; OC % 8 != 0 runs a
 * direct conv. */
int tsn_conv1d(tsn_runtime *rt, int wdtype, const void *Wp, const float *bias, const float *x, float *y, uint32_t T,
               uint32_t OL, uint32_t IC, uint32_t OC, uint32_t K, uint32_t stride, uint32_t pad, uint32_t dil,
               int convt);
/* elementwise, f32 (src/net.h:37-49; shaders/ops_conv.metal:9-57,193-201) */
int tsn_silu(tsn_runtime *rt, float *x, size_t n);
int tsn_copy(tsn_runtime *rt, const float *x, float *y, size_t n);
int tsn_swiglu(tsn_runtime *rt, const float *a, const float *b, float *y, size_t n);
int tsn_add(tsn_runtime *rt, const float *a, const float *b, float *y, size_t n);
int tsn_add_bcast_col(tsn_runtime *rt, const float *x, const float *v, float *y, uint32_t S, uint32_t H);
int tsn_cfg_euler(tsn_runtime *rt, const float *fc, const float *fu, float *x, size_t n, float cfg, float dt);
int tsn_geglu(tsn_runtime *rt, const float *a, const float *b, float *y, size_t n);   /* gelu_tanh(a)·b  :15-24 */
int tsn_gelu_quick(tsn_runtime *rt, float *x, size_t n);                              /* in place       :25-29 */
/* norms over rows of H floats, biased variance (shaders/ops_conv.metal:77-113). ln_wb and rms_w take
 * H % 4 == 0, H <= 2048 and 16-byte aligned rows. */
int tsn_ln_plain(tsn_runtime *rt, const float *x, float *y, uint32_t S, uint32_t H, float eps);
int tsn_ln_wb(tsn_runtime *rt, const float *x, float *y, const float *w, const float *b, uint32_t S, uint32_t H,
              float eps);
int tsn_rms_w(tsn_runtime *rt, const float *x, float *y, const float *w, uint32_t S, uint32_t H, float eps);
/* y[c] = mean over the S rows of x[:, c], rows summed in order. Runtime::mean_cols src/net.h:50,
 * shaders/ops_conv.metal:171-193 */
int tsn_mean_cols(tsn_runtime *rt, const float *x, float *y, uint32_t S, uint32_t H);
/* named kernels dispatched by dit_fwd.cpp (src/dit_fwd.cpp:16-22), as runtime launchers here:
 * adaln_ln  — AD{H,per_row,chunks,base,eps}  shaders/ops_conv.metal:127-144 (y f32 or f16)
 * gate_add  — GA{H,per_row,chunks,gate_idx}  shaders/ops_conv.metal:146-154
 * rms_head  — RH{ld,hd,col_off,row_off,eps}  shaders/ops_conv.metal:115-125 (in place)
 * rope_pairs— RP{ld,hd,col_off,row_off,fscale,base} shaders/ops_conv.metal:156-169 (in place)
 * attention — AttnP (src/gpu.h:60-70), src/dit_fwd.cpp:83-102; hd must be 64 */
int tsn_adaln_ln(tsn_runtime *rt, const float *x, const float *mod, void *y, int ydtype, uint32_t rows, uint32_t H,
                 uint32_t per_row, uint32_t chunks, uint32_t base, float eps);
int tsn_gate_add(tsn_runtime *rt, const float *x, const float *f, const float *mod, float *y, uint32_t rows,
                 uint32_t H, uint32_t per_row, uint32_t chunks, uint32_t gate_idx);
/* qkv_split3 — QS3{H,row_off}  shaders/ops_conv.metal:60-74: the element-interleaved projection rows
 * [rows][3H] (column 3c + j) -> block q|k|v rows row_off.. of dst [.][3H] (src/dit_fwd.cpp:33-36) */
int tsn_qkv_split3(tsn_runtime *rt, const float *src, float *dst, uint32_t rows, uint32_t H, uint32_t row_off);
int tsn_rms_head(tsn_runtime *rt, float *x, const float *w, uint32_t rows, uint32_t nh, uint32_t ld, uint32_t hd,
                 uint32_t col_off, uint32_t row_off, float eps);
int tsn_rope_pairs(tsn_runtime *rt, float *x, const int32_t *pos, uint32_t rows, uint32_t nh, uint32_t ld,
                   uint32_t hd, uint32_t col_off, uint32_t row_off, float fscale, float base);
int tsn_attention(tsn_runtime *rt, const float *qkv, float *out, uint32_t S, uint32_t nh, uint32_t hd, uint32_t ld,
                  uint32_t ldo, uint32_t q_off, uint32_t k_off, uint32_t v_off, uint32_t o_off, float scale);

/* Calibration (no reference counterpart: it measures the denominators a roofline is quoted
 * against). Sustained dense f16 MFMA rate (about 20 ms of one workgroup of 8 waves per CU running
 * independent v_mfma_f32_16x16x32_f16 chains), and device copy bandwidth (read + write of 1 GiB), both timed with
 * HIP events on the runtime's stream. Allocates and frees 2 GiB of device memory. */
int tsn_probe_peaks(tsn_runtime *rt, double *mfma_tflops, double *hbm_gbs);

/* ---------------- model: tn::DitModel (src/models.h:55-85) ---------------- */
typedef struct {
    int B;              /* batch: CFG arms folded in (sample 2p cond, 2p+1 uncond); 1, 2, 4, 8 or 16 */
    int La, Lt;         /* audio (latent) rows and text rows per sample */
    int H, NH, HD, F;   /* hidden 1024, heads 16, head dim 64, FFN width 4096 */
    int latent;         /* latent channels (64) */
    int temb_dim;       /* timestep sinusoid width (256) */
    int n_joint;        /* joint two-stream blocks (7) */
    int n_fused;        /* fused single-stream blocks over La+Lt rows (14) */
    int audio_ffn_conv; /* 1: audio FFN of joint blocks is conv1d k=3 pad=1 */
    float rope_theta;   /* 10000 */
    float t_max_period; /* timestep sinusoid max period (1): fr_k = (1e4/max_period)*1e4^(-2k/D) */
    float ln_eps;       /* 1e-5 (src/dit_fwd.cpp:29) */
    float rms_eps;      /* 1e-6 (src/dit_fwd.cpp:37) */
} tsn_dit_spec;

/* Spec of a workload: 0 one joint block (B=2, La=256), 1 one eval 8 s (B=2, La=256, Lt=141),
 * 2 sampler 8 s (as 1), 3 sampler 30 s (La=960), 4 batch 16 at 8 s. */
int tsn_dit_default_spec(int workload, tsn_dit_spec *out);
/* weight manifest (the flat BF16 weight buffer order) */
int tsn_dit_manifest_count(const tsn_dit_spec *spec);
int tsn_dit_manifest_entry(const tsn_dit_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                           int64_t *offset);
int64_t tsn_dit_manifest_total(const tsn_dit_spec *spec);

int tsn_dit_create(tsn_runtime *rt, const tsn_dit_spec *spec, tsn_dit **out);   /* DitModel::load src/dit.cpp:29-47 */
int tsn_dit_destroy(tsn_dit *dit);
/* WeightSet::load (src/net.mm:126-173) for the synthetic checkpoint: flat BF16, manifest order */
int tsn_dit_upload_weights(tsn_dit *dit, const uint16_t *weights_host, size_t numel);
/* One velocity evaluation. DitModel::forward (src/models.h:83-84, src/dit_fwd.cpp:104-304) with the
 * arms batched: z [B][La][latent], text [B][Lt][H], pooled [B][H] -> v [B][La][latent]; every
 * sample uses timestep t. Enqueued; call tsn_sync / tsn_commit before reading v. */
int tsn_dit_forward(tsn_dit *dit, const float *z, float t, const float *text, const float *pooled, float *v);
/* same with per-sample t (device [B]) and optional taps: X after each block, [n_blocks][B][La+Lt][H] */
int tsn_dit_forward_ex(tsn_dit *dit, const float *z, const float *t, const float *text, const float *pooled,
                       float *v, float *taps);
/* one joint / fused block on X [B][La+Lt][H] in place; g [B][H] is the global conditioning (silu inside) */
int tsn_dit_joint_block(tsn_dit *dit, int block, float *X, const float *g);
int tsn_dit_fused_block(tsn_dit *dit, int block, float *X, const float *g);
/* Rectified-flow Euler sampler with CFG (src/pipeline.cpp:141-155): x [B/2][La][latent] in/out */
int tsn_dit_sample(tsn_dit *dit, float *x, const float *text, const float *pooled, int steps, float cfg);
/* hipGraph capture of one forward (t read from device t[B]) or of the whole sampler, then replay */
int tsn_dit_capture_forward(tsn_dit *dit, const float *z, const float *t, const float *text, const float *pooled,
                            float *v);
int tsn_dit_capture_sample(tsn_dit *dit, float *x, const float *text, const float *pooled, int steps, float cfg);
int tsn_dit_replay(tsn_dit *dit);

/* Observability (no reference counterpart: the reference times only whole command buffers,
 * src/gpu.mm:168-174). One eager evaluation with a HIP event pair around every launch on the
 * runtime's stream; per kernel symbol: launches, summed ms, algorithmic flops and HBM bytes. */
typedef struct {
    char name[64];
    int launches;
    double total_ms;
    double flops;
    double bytes;
} tsn_kernel_stat;
int tsn_dit_profile_forward(tsn_dit *dit, const float *z, const float *t, const float *text, const float *pooled,
                            float *v, tsn_kernel_stat *stats, int cap, int *n_stats);

/* ---------------- model: the reference checkpoint's graph, tn::DitModel (src/models.h:55-85) ----------------
 * The three-stream graph of src/dit_fwd.cpp:104-304: latent (T rows, RoPE), clip (C rows, RoPE
 * positions scaled by T/C), text (TS rows, no RoPE); per-row adaLN of the latent stream from
 * extended_c = sync_gather + global_c (global_c = gcmlp + t_emb), SwiGLU FFNs (conv k3 for latent
 * and clip, linear for text), conv k3 out-projection for latent and clip, pre-only last joint
 * block, fused blocks over the latent rows alone, conv k7 final layer. CFG arms are folded into
 * the batch (sample 2p cond, 2p+1 uncond). */
typedef struct {
    int B;              /* batch; 1, 2, 4, 8 or 16 */
    int T;              /* latent rows: llround(44100/2048 * dur) (src/models.h:20-22); 172 at 8 s */
    int C;              /* clip rows: 8 * dur (src/pipeline.cpp:82) */
    int TS;             /* text rows (154) */
    int H, NH, HD, F;   /* hidden 1024, heads 16, head dim 64, SwiGLU width H_ffn 2816 (src/models.h:58-60) */
    int latent;         /* latent channels (64) */
    int n_joint;        /* joint three-stream blocks, the last one pre-only (7) */
    int n_fused;        /* fused blocks over the latent rows (14) */
    float rope_theta;   /* 10000 */
    float t_max_period; /* 1: timestep sinusoid fr_k = (1e4/max_period)*1e4^(-2k/H) (src/dit_fwd.cpp:111-118) */
    float ln_eps;       /* 1e-5 */
    float rms_eps;      /* 1e-6 */
} tsn_refdit_spec;
typedef struct tsn_refdit tsn_refdit;

/* geometry of a dur-second generation with B samples (src/pipeline.cpp:81-83) */
int tsn_refdit_spec_for_duration(int dur_s, int B, tsn_refdit_spec *out);
/* checkpoint tensor manifest (flat BF16 buffer order), the names DitModel::forward looks up with
 * W->need (src/dit_fwd.cpp); qkv weight/bias rows are element-interleaved as in the checkpoint */
int tsn_refdit_manifest_count(const tsn_refdit_spec *spec);
int tsn_refdit_manifest_entry(const tsn_refdit_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                              int64_t *offset);
int64_t tsn_refdit_manifest_total(const tsn_refdit_spec *spec);
int tsn_refdit_create(tsn_runtime *rt, const tsn_refdit_spec *spec, tsn_refdit **out);   /* DitModel::load src/dit.cpp:29-47 */
int tsn_refdit_destroy(tsn_refdit *dit);
/* WeightSet::load (src/net.mm:126-173): flat BF16 in manifest order; upload-time transforms:
 * qkv row de-interleave (replaces qkv_split3, src/dit_fwd.cpp:33-36), conv [OC][IC][K] -> [OC][K][IC],
 * BF16 -> FP16 */
int tsn_refdit_upload_weights(tsn_refdit *dit, const uint16_t *weights_host, size_t numel);
/* the same from an f32 buffer (dequantized checkpoint tensors, manifest order) */
int tsn_refdit_upload_weights_f32(tsn_refdit *dit, const float *weights_host, size_t numel);
/* DitModel::load (src/dit.cpp:29-47) + WeightSet::load (src/net.mm:126-173): every tensor of the
 * manifest looked up by name in a GGUF file, dequantized on the host (F32, F16, BF16, Q8_0), GEMM and
 * GEMV weights converted to f16 with the reference's rounding (src/net.mm:144-164) */
int tsn_refdit_load_gguf(tsn_refdit *dit, const char *path);
/* hyperparameters from the checkpoint's dit.* metadata and the SwiGLU width from the first latent
 * FFN weight (src/dit.cpp:32-43); B, T, C, TS are the caller's geometry */
int tsn_refdit_spec_from_gguf(const char *path, int B, int T, int C, int TS, tsn_refdit_spec *out);
/* DitModel::forward (src/models.h:83-84, src/dit_fwd.cpp:104-304) with the arms batched:
 * x [B][T][latent], clip_pp [B][C][H], text_pp [B][TS][H], gcmlp [B][H], sync_gather [B][T][H]
 * -> flow [B][T][latent]; every sample at flow time t. Enqueued; tsn_sync before reading flow. */
int tsn_refdit_forward(tsn_refdit *dit, const float *x, float t, const float *clip_pp, const float *text_pp,
                       const float *gcmlp, const float *sync_gather, float *flow);
/* same with per-sample t (device [B]) and optional taps: the streams [B][T+C+TS][H] after each block */
int tsn_refdit_forward_ex(tsn_refdit *dit, const float *x, const float *t, const float *clip_pp, const float *text_pp,
                          const float *gcmlp, const float *sync_gather, float *flow, float *taps);
/* Euler sampler with CFG (src/pipeline.cpp:141-155): x [B/2][T][latent] in/out */
int tsn_refdit_sample(tsn_refdit *dit, float *x, const float *clip_pp, const float *text_pp, const float *gcmlp,
                      const float *sync_gather, int steps, float cfg);
/* hipGraph capture of one forward (t from device t[B]) or of the whole sampler, then replay */
int tsn_refdit_capture_forward(tsn_refdit *dit, const float *x, const float *t, const float *clip_pp,
                               const float *text_pp, const float *gcmlp, const float *sync_gather, float *flow);
int tsn_refdit_capture_sample(tsn_refdit *dit, float *x, const float *clip_pp, const float *text_pp,
                              const float *gcmlp, const float *sync_gather, int steps, float cfg);
int tsn_refdit_replay(tsn_refdit *dit);
/* per-kernel statistics of one eager forward (no reference counterpart, as tsn_dit_profile_forward) */
int tsn_refdit_profile_forward(tsn_refdit *dit, const float *x, const float *t, const float *clip_pp,
                               const float *text_pp, const float *gcmlp, const float *sync_gather, float *flow,
                               tsn_kernel_stat *stats, int cap, int *n_stats);

/* ---------------- conditioning prep: DitModel::prep_conditioning / prep_text_arm (src/dit.cpp:55-191) ----------------
 * Once per generation (sync and clip streams) and once per CFG arm (text): the inputs of
 * tsn_refdit_forward. All GEMMs read f32-accurate f16 hi|lo operands. */
typedef struct {
    int H, F;           /* hidden 1024, SwiGLU width 2816 */
    int T, C, sync_S;   /* latent rows, clip rows (8/s), sync rows (24/s: src/pipeline.cpp:81-83) */
    int TS;             /* text rows (154) */
    int sync_dim, clip_dim, text_dim, gtext_dim;   /* input widths 768, 1024, 2048, 1024 */
} tsn_refcond_spec;
typedef struct tsn_refcond tsn_refcond;
int tsn_refcond_spec_for_duration(int dur_s, tsn_refcond_spec *out);
/* widths from a checkpoint (dit.hidden_dim; F and the input widths from the projections' shapes) */
int tsn_refcond_spec_from_gguf(const char *path, int T, int C, int sync_S, int TS, tsn_refcond_spec *out);
int tsn_refcond_manifest_count(const tsn_refcond_spec *spec);
int tsn_refcond_manifest_entry(const tsn_refcond_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                               int64_t *offset);
int64_t tsn_refcond_manifest_total(const tsn_refcond_spec *spec);
int tsn_refcond_create(tsn_runtime *rt, const tsn_refcond_spec *spec, tsn_refcond **out);
int tsn_refcond_destroy(tsn_refcond *c);
int tsn_refcond_upload_weights(tsn_refcond *c, const uint16_t *weights_host, size_t numel);   /* flat BF16 */
int tsn_refcond_upload_weights_f32(tsn_refcond *c, const float *weights_host, size_t numel);
int tsn_refcond_load_gguf(tsn_refcond *c, const char *path);   /* WeightSet::load, src/net.mm:126-173 */
/* DitModel::prep_conditioning (src/dit.cpp:55-135): clip_f [C][clip_dim], sync_f [sync_S][sync_dim]
 * -> clip_pp [C][H], sync_gather [T][H], clip_fc [H] (device pointers) */
int tsn_refcond_prep_conditioning(tsn_refcond *c, const float *clip_f, const float *sync_f, float *clip_pp,
                                  float *sync_gather, float *clip_fc);
/* DitModel::prep_text_arm (src/dit.cpp:137-191): text_cat [TS][text_dim], gtext [gtext_dim], clip_fc [H]
 * -> text_pp [TS][H], gcmlp [H] */
int tsn_refcond_prep_text_arm(tsn_refcond *c, const float *text_cat, const float *gtext, const float *clip_fc,
                              float *text_pp, float *gcmlp);

/* ---------------- VAE decoder: tn::VaeModel (src/models.h:87-94, src/vae.cpp:17-86) ----------------
 * latent [T][64] -> conv k7 (+b) -> 5 stages { snake -> transposed conv (stride s, kernel 2s, +b)
 * -> 3 residual units (dilation 1, 3, 9) } -> snake -> conv k7 (no bias) -> audio [T*prod(s)][2].
 * f32 in the reference (src/vae.cpp:12); here every GEMM is f32-accurate on f16 MFMA (three products
 * of a hi/lo split of both operands), the residual stream f32. */
typedef struct {
    int T, latent;   /* latent rows (llround(44100/2048*dur), src/models.h:16-21) and width 64 */
    int width[6];    /* input conv output width, then each stage's output width: 2048,1024,512,256,128,128 */
    int stride[5];   /* upsampling factors 8, 8, 4, 4, 2 (src/vae.cpp:20) */
    int kt[5];       /* transposed-conv kernel sizes (2*stride in the checkpoint) */
    int out_ch;      /* audio channels (2) */
} tsn_vae_spec;
typedef struct tsn_vae tsn_vae;
int tsn_vae_spec_for_duration(int dur_s, tsn_vae_spec *out);
/* widths and kernel sizes from a checkpoint's tensor shapes (vae-f32.gguf); T from the caller */
int tsn_vae_spec_from_gguf(const char *path, int T, tsn_vae_spec *out);
int64_t tsn_vae_audio_len(const tsn_vae_spec *spec);   /* T_audio = T * prod(stride) */
int tsn_vae_manifest_count(const tsn_vae_spec *spec);
int tsn_vae_manifest_entry(const tsn_vae_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                           int64_t *offset);
int64_t tsn_vae_manifest_total(const tsn_vae_spec *spec);
int tsn_vae_create(tsn_runtime *rt, const tsn_vae_spec *spec, tsn_vae **out);   /* VaeModel::load src/vae.cpp:10-15 */
int tsn_vae_destroy(tsn_vae *v);
int tsn_vae_upload_weights(tsn_vae *v, const float *weights_host, size_t numel);   /* flat f32, manifest order */
int tsn_vae_load_gguf(tsn_vae *v, const char *path);   /* WeightSet::load(keep_f32), src/net.mm:126-173 */
/* VaeModel::decode (src/vae.cpp:17-86): latent [T][latent] -> audio [T_audio][out_ch], device pointers,
 * enqueued on the runtime's stream (the reference returns host audio; download it with tsn_download) */
int tsn_vae_decode(tsn_vae *v, const float *latent, float *audio);
int tsn_vae_capture_decode(tsn_vae *v, const float *latent, float *audio);   /* hipGraph of one decode */
int tsn_vae_replay(tsn_vae *v);
int tsn_vae_profile_decode(tsn_vae *v, const float *latent, float *audio, tsn_kernel_stat *stats, int cap,
                           int *n_stats);

/* ---------------- text encoders: tn::ClipModel, tn::T5Model (src/models.h:24-52) ----------------
 * f32 throughout, as the reference loads both (src/clip.cpp:7, src/t5.cpp:22): f32 MFMA GEMMs, f32
 * attention over the 77-token context. ids are host arrays (the reference's std::vector<int32_t>);
 * outputs are device pointers enqueued on the runtime's stream. */
typedef struct {
    int H, NL, NH, ctx, vocab;   /* 1024, 24 layers, 16 heads, 77 tokens, 49408 (clip.* metadata) */
    float eps;                   /* LayerNorm eps 1e-5 */
} tsn_clip_spec;
typedef struct {
    int d, d_ff, NL, NH, ctx, vocab;   /* 2048, 5120, 24 layers, 32 heads, 77, 32128 (t5.* metadata) */
    int n_bucket, max_dist;            /* relative-position buckets 32, max distance 128 */
    float eps;                         /* RMSNorm eps 1e-6 */
} tsn_t5_spec;
typedef struct tsn_clip tsn_clip;
typedef struct tsn_t5 tsn_t5;
int tsn_clip_spec_default(tsn_clip_spec *out);
int tsn_clip_spec_from_gguf(const char *path, tsn_clip_spec *out);   /* ClipModel::load src/clip.cpp:6-32 */
int tsn_clip_manifest_count(const tsn_clip_spec *spec);
int tsn_clip_manifest_entry(const tsn_clip_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                            int64_t *offset);
int64_t tsn_clip_manifest_total(const tsn_clip_spec *spec);
int tsn_clip_create(tsn_runtime *rt, const tsn_clip_spec *spec, tsn_clip **out);
int tsn_clip_destroy(tsn_clip *c);
int tsn_clip_upload_weights(tsn_clip *c, const float *weights_host, size_t numel);   /* flat f32, manifest order */
int tsn_clip_load_gguf(tsn_clip *c, const char *path);
/* ClipModel::encode (src/clip.cpp:34-92): ids [ctx] -> per_token [ctx][H], global [H] */
int tsn_clip_encode(tsn_clip *c, const int32_t *ids_host, float *per_token, float *global);
int tsn_clip_profile_encode(tsn_clip *c, const int32_t *ids_host, float *per_token, float *global,
                            tsn_kernel_stat *stats, int cap, int *n_stats);
int tsn_t5_spec_default(tsn_t5_spec *out);
int tsn_t5_spec_from_gguf(const char *path, tsn_t5_spec *out);   /* T5Model::load src/t5.cpp:21-55 */
int tsn_t5_manifest_count(const tsn_t5_spec *spec);
int tsn_t5_manifest_entry(const tsn_t5_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                          int64_t *offset);
int64_t tsn_t5_manifest_total(const tsn_t5_spec *spec);
int tsn_t5_create(tsn_runtime *rt, const tsn_t5_spec *spec, tsn_t5 **out);
int tsn_t5_destroy(tsn_t5 *t);
int tsn_t5_upload_weights(tsn_t5 *t, const float *weights_host, size_t numel);
int tsn_t5_load_gguf(tsn_t5 *t, const char *path);   /* Q8_0 / F16 / F32 tensors dequantized to f32 */
/* T5Model::encode (src/t5.cpp:88-131): ids [ctx] -> out [ctx][d] */
int tsn_t5_encode(tsn_t5 *t, const int32_t *ids_host, float *out);
int tsn_t5_profile_encode(tsn_t5 *t, const int32_t *ids_host, float *out, tsn_kernel_stat *stats, int cap,
                          int *n_stats);
/* the relative-position bucket of rel = key - query (t5_bucket, src/t5.cpp:6-19) */
int tsn_t5_bucket(int rel, int n_bucket, int max_dist);

/* ---------------- tokenizers: tn::ClipTokenizer, tn::T5Tokenizer (src/tokenizers.h:12-31) ----------------
 * Host only. Vocabularies come from the tokenizer GGUFs' array metadata. */
typedef struct tsn_clip_tokenizer tsn_clip_tokenizer;
typedef struct tsn_t5_tokenizer tsn_t5_tokenizer;
int tsn_clip_tokenizer_load(const char *path, tsn_clip_tokenizer **out);   /* ClipTokenizer::load */
int tsn_clip_tokenizer_destroy(tsn_clip_tokenizer *t);
/* ClipTokenizer::encode: writes exactly ctx ids (bos, BPE tokens, eos, eos padding) */
int tsn_clip_tokenizer_encode(const tsn_clip_tokenizer *t, const char *text, int ctx, int32_t *ids);
int tsn_t5_tokenizer_load(const char *path, tsn_t5_tokenizer **out);   /* T5Tokenizer::load */
int tsn_t5_tokenizer_destroy(tsn_t5_tokenizer *t);
/* T5Tokenizer::encode: up to ctx ids (pad != 0 pads with pad_id to ctx); *n_ids = count written */
int tsn_t5_tokenizer_encode(const tsn_t5_tokenizer *t, const char *text, int ctx, int pad, int32_t *ids,
                            int *n_ids);

/* ---------------- GGUF checkpoint reader: tn::GgufFile / tn::to_f32 (src/gguf.h:42-86) ----------------
 * mmap, GGUF v2/v3, typed metadata, tensor infos with ne[0] fastest, data at general.alignment. */
typedef struct tsn_gguf tsn_gguf;
int tsn_gguf_open(const char *path, tsn_gguf **out);                 /* GgufFile::open src/gguf.h:48 */
int tsn_gguf_close(tsn_gguf *g);                                     /* GgufFile::~GgufFile src/gguf.h:47 */
int tsn_gguf_tensor_count(const tsn_gguf *g);                        /* GgufFile::n_tensors src/gguf.h:59 */
/* name, GGML type (0 F32, 1 F16, 8 Q8_0, 30 BF16), n_dims, ne[4] (GgufTensor, src/gguf.h:32-40) */
int tsn_gguf_tensor_info(const tsn_gguf *g, int idx, char *name, int name_cap, uint32_t *type, uint32_t *n_dims,
                         uint64_t *ne4);
/* to_f32 (src/gguf.h:85): F16 and Q8_0 scales with subnormals flushed to zero, as the reference */
int tsn_gguf_tensor_to_f32(const tsn_gguf *g, const char *name, float *out_host, size_t cap);
int64_t tsn_gguf_get_i64(const tsn_gguf *g, const char *key, int64_t def);   /* GgufFile::get_i64 src/gguf.h:53 */
double tsn_gguf_get_f64(const tsn_gguf *g, const char *key, double def);    /* GgufFile::get_f64 src/gguf.h:54 */

/* ---------------- synthetic data (specified generator; see thinksound-native_amd/csrc/synth.cpp) ---------------- */
int tsn_synth_normal_f32(uint64_t seed, uint64_t index, double mean, double std, size_t n, float *out_host);
int tsn_synth_normal_bf16(uint64_t seed, uint64_t index, double mean, double std, size_t n, uint16_t *out_host);
int tsn_synth_uniform_f32(uint64_t seed, uint64_t index, double lo, double hi, size_t n, float *out_host);
/* all weights of a spec, flat BF16 in manifest order: N(0, 0.02); q/k norm weights N(norm_mean, 0.02) */
int tsn_dit_synth_weights(const tsn_dit_spec *spec, uint64_t seed, double norm_mean, uint16_t *out_host);
int tsn_refdit_synth_weights(const tsn_refdit_spec *spec, uint64_t seed, double norm_mean, uint16_t *out_host);
int tsn_refcond_synth_weights(const tsn_refcond_spec *spec, uint64_t seed, uint16_t *out_host);
/* VAE: conv weights N(0, 1/(IC*K)) (residual-branch k1 convs N(0, 0.25/IC)), biases N(0, 0.02), snake
 * alpha and beta N(0, 0.1); f32 */
int tsn_vae_synth_weights(const tsn_vae_spec *spec, uint64_t seed, float *out_host);
/* text encoders: embeddings N(0, 1), norm weights 1 + N(0, 0.1), biases N(0, 0.02), projections into the
 * residual stream N(0, 0.25/fan_in), other linear weights N(0, 1/fan_in), T5 relative bias N(0, 0.25); f32 */
int tsn_clip_synth_weights(const tsn_clip_spec *spec, uint64_t seed, float *out_host);
int tsn_t5_synth_weights(const tsn_t5_spec *spec, uint64_t seed, float *out_host);

#ifdef __cplusplus
}
#endif

#endif /* TSN_H */
