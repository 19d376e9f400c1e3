// oracle.h — CPU f32 restatement of the ThinkSound-native DiT velocity path.
//
// TEST INFRASTRUCTURE ONLY. This library is the checker: only tests/, the smoke
// entry point and the benchmark's CPU-baseline leg load it. The product library
// (libtsn) never links, loads or calls it.
//
// Every function restates the reference's op semantics in plain f32 arithmetic on
// the host (citations are path:line into the ThinkSound-native sources). Reductions
// run in a fixed order per output element, so results do not depend on the OpenMP
// thread count. Pinning of each function (closed forms, brute force, invariants) is
// done by tests/test_oracle.py; every function below is pinned there.
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- single ops ---------------- */

// Y[m*ldy+n] = sum_k X[m*ldx+k] * W[n*ldw+k] (+ bias[n])
// Follows shaders/gemm_mpp.metal:2-3,39-46 (Y = X·Wᵀ + b) and src/net.mm:14-23 (ld defaults).
void orc_gemm(const float *W, const float *X, float *Y, const float *bias,
              int M, int N, int K, int ldx, int ldw, int ldy);

// y[n] = bias[n] + sum_k W[n*ldw+k] * x[k]        (shaders/gemm_attn.metal:47-74)
void orc_gemv(const float *W, const float *x, float *y, const float *bias, int N, int K, int ldw);

// conv1d, x [T,IC] row-major, y [OL,OC] row-major, W [OC][IC][K] (reference layout),
// ti = t*stride - pad + k*dil, zero outside [0,T).   (shaders/ops_conv.metal:221-246,262-283;
// src/net.mm:25-49). Computed as im2col + gemm, the reference's own route.
void orc_conv1d(const float *W, const float *bias, const float *x, float *y,
                int T, int OL, int IC, int OC, int K, int stride, int pad, int dil);

// Direct (non-im2col) conv1d, same semantics; used to cross-check orc_conv1d.
void orc_conv1d_direct(const float *W, const float *bias, const float *x, float *y,
                       int T, int OL, int IC, int OC, int K, int stride, int pad, int dil);

// y = LN(x; eps, no affine)*(1 + m[base+H+i]) + m[base+i], biased variance, two-pass.
// m = mod + (per_row ? row*chunks*H : 0).             (shaders/ops_conv.metal:127-144)
void orc_adaln_ln(const float *x, const float *mod, float *y, int rows, int H,
                  int per_row, int chunks, int base, float eps);

// y = x + f * m[gate_idx*H + c], m per row or broadcast. (shaders/ops_conv.metal:146-154)
void orc_gate_add(const float *x, const float *f, const float *mod, float *y, int rows, int H,
                  int per_row, int chunks, int gate_idx);

// in-place per-head RMSNorm on a column slice: r = r*rsqrt(mean(r^2)+eps)*w[i]
// r = x + (row_off+row)*ld + col_off + head*hd.          (shaders/ops_conv.metal:115-125)
void orc_rms_head(float *x, const float *w, int rows, int nh, int ld, int hd,
                  int col_off, int row_off, float eps);

// in-place interleaved-pair RoPE: inv = base^(-2j/hd), ang = pos*fscale*inv
// (pos = row when pos == NULL).                          (shaders/ops_conv.metal:156-169)
void orc_rope_pairs(float *x, const int32_t *pos, int rows, int nh, int ld, int hd,
                    int col_off, int row_off, float fscale, float base);

// non-causal attention over a [S, ld] qkv buffer: O[q, o_off+h*hd+d] = softmax_k(scale*Q·K)·V
// Materialised scores, max-subtracted exp, normalise.    (shaders/gemm_attn.metal:96-202,
// src/dit_fwd.cpp:83-102)
void orc_attention(const float *qkv, float *out, int S, int nh, int hd, int ld, int ldo,
                   int q_off, int k_off, int v_off, int o_off, float scale);

// elementwise ops (shaders/ops_conv.metal:9-13,30-57,193-201)
void orc_silu(float *x, size_t n);
void orc_swiglu(const float *a, const float *b, float *y, size_t n);
void orc_add(const float *a, const float *b, float *y, size_t n);
void orc_add_bcast_col(const float *x, const float *v, float *y, int S, int H);
void orc_cfg_euler(const float *fc, const float *fu, float *x, size_t n, float cfg, float dt);

// the rest of the reference's launcher surface (src/net.h:37-50; shaders/ops_conv.metal:15-29,60-89,171-193):
// gated tanh-GELU y = gelu_tanh(a)*b (argument clamped to [-10, 10]); quick GELU in place; LayerNorm
// without affine over rows of H; column means over S rows; qkv de-interleave into rows row_off..
void orc_geglu(const float *a, const float *b, float *y, size_t n);
void orc_gelu_quick(float *x, size_t n);
void orc_ln_plain(const float *x, float *y, int S, int H, float eps);
void orc_mean_cols(const float *x, float *y, int S, int H);
void orc_qkv_split3(const float *src, float *dst, int rows, int H, int row_off);

// sinusoidal timestep embedding, cos half then sin half:
// fr_k = (10000/max_period) * 10000^(-2k/D); out[k] = cos(t*fr_k), out[D/2+k] = sin(t*fr_k)
// (src/dit_fwd.cpp:111-119)
void orc_timestep_embedding(float t, int D, float max_period, float *out);

/* ---------------- block graph ---------------- */

// Graph spec. Field meaning mirrors the library's tsn_dit_spec.
typedef struct {
    int B, La, Lt;          // batch (CFG arms folded), audio rows, text rows
    int H, NH, HD, F;       // hidden, heads, head dim, FFN width
    int latent, temb_dim;   // latent channels, timestep sinusoid width
    int n_joint, n_fused;   // joint blocks, fused single-stream blocks
    int audio_ffn_conv;     // 1: audio FFN is conv1d k=3 pad=1 (joint blocks)
    float rope_theta, t_max_period, ln_eps, rms_eps;
} orc_spec;

// Number of tensors in the weight manifest and the element count / offset of each,
// in manifest order (the library's manifest must agree; tests check it).
int orc_manifest_count(const orc_spec *s);
int64_t orc_manifest_numel(const orc_spec *s, int idx);
int64_t orc_manifest_total(const orc_spec *s);
// Name of tensor idx written into buf (NUL-terminated, truncated to cap).
void orc_manifest_name(const orc_spec *s, int idx, char *buf, int cap);

// One joint block on X [B, La+Lt, H] (audio rows first per sample) in place;
// gs = silu(g) [B, H] feeds the adaLN modulation.
void orc_joint_block(const orc_spec *s, const float *weights, int block, float *X, const float *gs);

// One fused single-stream block on X [B, S, H] in place.
void orc_fused_block(const orc_spec *s, const float *weights, int block, float *X, const float *gs);

// One full velocity evaluation.
//   z [B, La, latent], t [B], text [B, Lt, H], pooled [B, H]  ->  v [B, La, latent]
//   taps (optional, may be NULL): X [B, S, H] after each of the n_joint+n_fused blocks.
//   gs_out (optional): silu(global cond) [B, H].
void orc_dit_forward(const orc_spec *s, const float *weights, const float *z, const float *t,
                     const float *text, const float *pooled, float *v, float *taps, float *gs_out);

// Rectified-flow Euler sampler with CFG (src/pipeline.cpp:141-155). B = 2*P: sample 2p is the
// conditional arm and 2p+1 the unconditional arm of prompt p. x [P, La, latent] in/out.
// t_s = 1 - s/steps, dt = t_{s+1} - t_s; x += dt*(v_u + cfg*(v_c - v_u)).
void orc_dit_sample(const orc_spec *s, const float *weights, float *x, const float *text,
                    const float *pooled, int steps, float cfg);

/* ---------------- the reference's own three-stream graph (oracle_ref.cpp) ---------------- */

// B samples (CFG arms), T latent rows, C clip rows, TS text rows; F = SwiGLU width (H_ffn);
// the timestep sinusoid is H wide; the last joint block is pre-only.
typedef struct {
    int B, T, C, TS;
    int H, NH, HD, F;
    int latent;
    int n_joint, n_fused;
    float rope_theta, t_max_period, ln_eps, rms_eps;
} orc_ref_spec;

int orc_ref_manifest_count(const orc_ref_spec *s);
int64_t orc_ref_manifest_numel(const orc_ref_spec *s, int idx);
void orc_ref_manifest_name(const orc_ref_spec *s, int idx, char *buf, int cap);

// One velocity evaluation of the reference graph per sample (src/dit_fwd.cpp:104-304):
//   x [B, T, latent], t [B], clip_pp [B, C, H], text_pp [B, TS, H], gcmlp [B, H],
//   sync_gather [B, T, H]  ->  v [B, T, latent];
//   taps (optional): the joint state [B, T+C+TS, H] (latent, clip, text rows) after each block.
void orc_ref_dit_forward(const orc_ref_spec *s, const float *weights, const float *x, const float *t,
                         const float *clip_pp, const float *text_pp, const float *gcmlp,
                         const float *sync_gather, float *v, float *taps);

// CFG Euler sampler over the reference graph: sample 2p cond, 2p+1 uncond; x [B/2, T, latent].
void orc_ref_dit_sample(const orc_ref_spec *s, const float *weights, float *x, const float *clip_pp,
                        const float *text_pp, const float *gcmlp, const float *sync_gather, int steps,
                        float cfg);

/* ---------------- the reference's conditioning prep (oracle_cond.cpp) ---------------- */

// H hidden, F SwiGLU width, T latent rows, C clip rows, sync_S sync rows, TS text rows; feature
// widths of the sync (768), clip (1024), text (2048) and pooled-text (1024) inputs
typedef struct {
    int H, F, T, C, sync_S, TS;
    int sync_dim, clip_dim, text_dim, gtext_dim;
} orc_refcond_spec;

int orc_refcond_manifest_count(const orc_refcond_spec *s);
int64_t orc_refcond_manifest_numel(const orc_refcond_spec *s, int idx);
void orc_refcond_manifest_name(const orc_refcond_spec *s, int idx, char *buf, int cap);

// DitModel::prep_conditioning (src/dit.cpp:55-135): clip_f [C, clip_dim], sync_f [sync_S, sync_dim]
//   -> clip_pp [C, H], sync_gather [T, H], clip_fc [H]
void orc_ref_prep_conditioning(const orc_refcond_spec *s, const float *weights, const float *clip_f,
                               const float *sync_f, float *clip_pp, float *sync_gather, float *clip_fc);
// DitModel::prep_text_arm (src/dit.cpp:137-191): text_cat [TS, text_dim], gtext [gtext_dim], clip_fc [H]
//   -> text_pp [TS, H], gcmlp [H]
void orc_ref_prep_text_arm(const orc_refcond_spec *s, const float *weights, const float *text_cat,
                           const float *gtext, const float *clip_fc, float *text_pp, float *gcmlp);

/* ---------------- the reference's VAE decoder (oracle_vae.cpp) ---------------- */

// T latent frames of `latent` channels; width[0] is the input conv's output width, width[n+1] the
// output width of upsampling stage n; stride[n] and kt[n] the stage's transposed-conv stride and
// kernel size; out_ch audio channels
typedef struct {
    int T, latent;
    int width[6];
    int stride[5];
    int kt[5];
    int out_ch;
} orc_vae_spec;

int orc_vae_manifest_count(const orc_vae_spec *s);
int64_t orc_vae_manifest_numel(const orc_vae_spec *s, int idx);
void orc_vae_manifest_name(const orc_vae_spec *s, int idx, char *buf, int cap);
int64_t orc_vae_audio_len(const orc_vae_spec *s);

// snake: y = x + sin(x*exp(alpha[c]))^2 * exp(-beta[c]), x and y [S, C] (shaders/ops_conv.metal:204-213)
void orc_snake(const float *x, float *y, const float *alpha, const float *beta, int S, int C);
// transposed conv in the reference's gather form (src/net.mm:36-48, shaders/ops_conv.metal:262-283):
// y[t, oc] = b[oc] + sum_{ic,k} x[(t-pad+k)/stride, ic] * W[oc][ic][k] over taps where t-pad+k >= 0
// is a multiple of stride and the row is inside [0, T)
void orc_conv1d_t(const float *W, const float *bias, const float *x, float *y, int T, int OL, int IC, int OC,
                  int K, int stride, int pad);
// VaeModel::decode (src/vae.cpp:17-86): latent [T, latent] -> audio [T*prod(stride), out_ch]
void orc_vae_decode(const orc_vae_spec *s, const float *weights, const float *latent, float *audio);

/* ---------------- the reference's text encoders (oracle_enc.cpp) ---------------- */

typedef struct { int H, NL, NH, ctx, vocab; float eps; } orc_clip_spec;
typedef struct { int d, d_ff, NL, NH, ctx, vocab, n_bucket, max_dist; float eps; } orc_t5_spec;

int orc_clip_manifest_count(const orc_clip_spec *s);
int64_t orc_clip_manifest_numel(const orc_clip_spec *s, int idx);
void orc_clip_manifest_name(const orc_clip_spec *s, int idx, char *buf, int cap);
int orc_t5_manifest_count(const orc_t5_spec *s);
int64_t orc_t5_manifest_numel(const orc_t5_spec *s, int idx);
void orc_t5_manifest_name(const orc_t5_spec *s, int idx, char *buf, int cap);
// LayerNorm with weight and bias (shaders/ops_conv.metal:90-103), RMSNorm with weight (:104-113)
void orc_ln_wb(const float *x, float *y, const float *w, const float *b, int rows, int H, float eps);
void orc_rms_w(const float *x, float *y, const float *w, int rows, int H, float eps);
// bidirectional relative-position bucket of rel = key - query (src/t5.cpp:6-19)
int orc_t5_bucket(int rel, int num_buckets, int max_dist);
// attention with the reference's bias modes (shaders/gemm_attn.metal:84-202): 1 T5 (pad keys
// masked, bucketed bias rel[bucket*nh + h]), 2 CLIP (k <= q and k <= eot), 0 none
void orc_enc_attention(const float *qkv, float *out, int S, int nh, int hd, int ld, int q_off, int k_off, int v_off,
                       int ldo, float scale, int mode, const int32_t *bucket, const float *rel, const int32_t *pad,
                       int eot);
// ClipModel::encode (src/clip.cpp:34-92): ids [ctx] -> per_token [ctx, H], global [H]
void orc_clip_encode(const orc_clip_spec *s, const float *weights, const int32_t *ids, float *per_token,
                     float *global);
// T5Model::encode (src/t5.cpp:88-131): ids [ctx] -> out [ctx, d]
void orc_t5_encode(const orc_t5_spec *s, const float *weights, const int32_t *ids, float *out);

// number of OpenMP threads the oracle uses (for the CPU-baseline report)
int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
