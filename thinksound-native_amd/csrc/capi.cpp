// capi.cpp — extern "C" boundary of libtsn (declarations and reference citations in include/tsn.h).
#include "../../include/tsn.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <functional>
#include <new>

#include "dit.h"
#include "encoders.h"
#include "gguf.h"
#include "refcond.h"
#include "refdit.h"
#include "tokenizers.h"
#include "vae.h"

namespace tsn {
void synth_normal_f32(uint64_t seed, uint64_t idx, double mean, double std, size_t n, float *out);
void synth_normal_bf16(uint64_t seed, uint64_t idx, double mean, double std, size_t n, uint16_t *out);
void synth_uniform_f32(uint64_t seed, uint64_t idx, double lo, double hi, size_t n, float *out);
}

struct tsn_runtime {
    tsn::Runtime rt;
};
struct tsn_dit {
    tsn::DitModel m;
};
struct tsn_refdit {
    tsn::RefDitModel m;
};
struct tsn_gguf {
    tsn::GgufReader r;
};
struct tsn_refcond {
    tsn::RefCondModel m;
};
struct tsn_vae {
    tsn::VaeModel m;
};
struct tsn_clip {
    tsn::ClipModel m;
};
struct tsn_t5 {
    tsn::T5Model m;
};
struct tsn_clip_tokenizer {
    tsn::ClipBpe t;
};
struct tsn_t5_tokenizer {
    tsn::T5Unigram t;
};

#define RT_CHECK(r)                                                 \
    do {                                                            \
        if (!(r)) { tsn::set_error("null runtime handle"); return TSN_ERR_ARG; } \
    } while (0)

static tsn::DitSpec to_spec(const tsn_dit_spec *c) {
    tsn::DitSpec s;
    s.B = c->B; s.La = c->La; s.Lt = c->Lt; s.H = c->H; s.NH = c->NH; s.HD = c->HD; s.F = c->F;
    s.latent = c->latent; s.temb_dim = c->temb_dim; s.n_joint = c->n_joint; s.n_fused = c->n_fused;
    s.audio_ffn_conv = c->audio_ffn_conv; s.rope_theta = c->rope_theta; s.t_max_period = c->t_max_period;
    s.ln_eps = c->ln_eps; s.rms_eps = c->rms_eps;
    return s;
}

static tsn::RefDitSpec to_ref_spec(const tsn_refdit_spec *c) {
    tsn::RefDitSpec s;
    s.B = c->B; s.T = c->T; s.C = c->C; s.TS = c->TS; s.H = c->H; s.NH = c->NH; s.HD = c->HD; s.F = c->F;
    s.latent = c->latent; s.n_joint = c->n_joint; s.n_fused = c->n_fused; s.rope_theta = c->rope_theta;
    s.t_max_period = c->t_max_period; s.ln_eps = c->ln_eps; s.rms_eps = c->rms_eps;
    return s;
}

static tsn::RefCondSpec to_cond_spec(const tsn_refcond_spec *c) {
    tsn::RefCondSpec s;
    s.H = c->H; s.F = c->F; s.T = c->T; s.C = c->C; s.sync_S = c->sync_S; s.TS = c->TS;
    s.sync_dim = c->sync_dim; s.clip_dim = c->clip_dim; s.text_dim = c->text_dim; s.gtext_dim = c->gtext_dim;
    return s;
}
static void from_cond_spec(const tsn::RefCondSpec &s, tsn_refcond_spec *c) {
    c->H = s.H; c->F = s.F; c->T = s.T; c->C = s.C; c->sync_S = s.sync_S; c->TS = s.TS;
    c->sync_dim = s.sync_dim; c->clip_dim = s.clip_dim; c->text_dim = s.text_dim; c->gtext_dim = s.gtext_dim;
}

static tsn::VaeSpec to_vae_spec(const tsn_vae_spec *c) {
    tsn::VaeSpec s;
    s.T = c->T; s.latent = c->latent; s.out_ch = c->out_ch;
    for (int i = 0; i < 6; ++i) s.width[i] = c->width[i];
    for (int i = 0; i < 5; ++i) { s.stride[i] = c->stride[i]; s.kt[i] = c->kt[i]; }
    return s;
}
static void from_vae_spec(const tsn::VaeSpec &s, tsn_vae_spec *c) {
    c->T = s.T; c->latent = s.latent; c->out_ch = s.out_ch;
    for (int i = 0; i < 6; ++i) c->width[i] = s.width[i];
    for (int i = 0; i < 5; ++i) { c->stride[i] = s.stride[i]; c->kt[i] = s.kt[i]; }
}

static tsn::ClipSpec to_clip_spec(const tsn_clip_spec *c) {
    return tsn::ClipSpec{c->H, c->NL, c->NH, c->ctx, c->vocab, c->eps};
}
static void from_clip_spec(const tsn::ClipSpec &s, tsn_clip_spec *c) {
    c->H = s.H; c->NL = s.NL; c->NH = s.NH; c->ctx = s.ctx; c->vocab = s.vocab; c->eps = s.eps;
}
static tsn::T5Spec to_t5_spec(const tsn_t5_spec *c) {
    return tsn::T5Spec{c->d, c->d_ff, c->NL, c->NH, c->ctx, c->vocab, c->n_bucket, c->max_dist, c->eps};
}
static void from_t5_spec(const tsn::T5Spec &s, tsn_t5_spec *c) {
    c->d = s.d; c->d_ff = s.d_ff; c->NL = s.NL; c->NH = s.NH; c->ctx = s.ctx; c->vocab = s.vocab;
    c->n_bucket = s.n_bucket; c->max_dist = s.max_dist; c->eps = s.eps;
}
static int manifest_entry(const std::vector<tsn::ManifestEntry> &m, int idx, char *name, int name_cap,
                          int64_t *numel, int64_t *offset) {
    if (idx < 0 || idx >= (int)m.size()) { tsn::set_error("manifest index out of range"); return TSN_ERR_ARG; }
    if (name && name_cap > 0) snprintf(name, (size_t)name_cap, "%s", m[idx].name.c_str());
    if (numel) *numel = m[idx].numel;
    if (offset) *offset = m[idx].offset;
    return TSN_OK;
}

static int copy_stats(const std::vector<tsn::KernelStat> &ks, tsn_kernel_stat *stats, int cap, int *n_stats) {
    const int n = (int)ks.size() < cap ? (int)ks.size() : cap;
    for (int i = 0; i < n; ++i) {
        snprintf(stats[i].name, sizeof stats[i].name, "%s", ks[i].name.c_str());
        stats[i].launches = ks[i].launches;
        stats[i].total_ms = ks[i].ms;
        stats[i].flops = ks[i].flops;
        stats[i].bytes = ks[i].bytes;
    }
    *n_stats = n;
    return TSN_OK;
}

extern "C" {

const char *tsn_last_error(void) { return tsn::last_error(); }
int tsn_version(void) { return 1; }

int tsn_runtime_create(int device, tsn_runtime **out) {
    if (!out) { tsn::set_error("null out pointer"); return TSN_ERR_ARG; }
    *out = nullptr;
    tsn_runtime *r = new (std::nothrow) tsn_runtime();
    if (!r) { tsn::set_error("out of host memory"); return TSN_ERR_OOM; }
    const int rc = r->rt.init(device);
    if (rc != TSN_OK) { delete r; return rc; }
    *out = r;
    return TSN_OK;
}
int tsn_runtime_destroy(tsn_runtime *rt) { delete rt; return TSN_OK; }
int tsn_alloc(tsn_runtime *rt, size_t bytes, void **dptr) { RT_CHECK(rt); return rt->rt.dev.alloc(bytes, dptr); }
int tsn_free(tsn_runtime *rt, void *dptr) { RT_CHECK(rt); return rt->rt.dev.free(dptr); }
int tsn_upload(tsn_runtime *rt, void *dptr, const void *src, size_t bytes) { RT_CHECK(rt); return rt->rt.dev.upload(dptr, src, bytes); }
int tsn_download(tsn_runtime *rt, void *dst, const void *dptr, size_t bytes) { RT_CHECK(rt); return rt->rt.dev.download(dst, dptr, bytes); }
int tsn_begin(tsn_runtime *rt) { RT_CHECK(rt); return rt->rt.dev.begin(); }
int tsn_commit(tsn_runtime *rt) { RT_CHECK(rt); return rt->rt.dev.commit(); }
double tsn_last_gpu_ms(tsn_runtime *rt) { return rt ? rt->rt.dev.last_gpu_ms() : -1.0; }
int tsn_sync(tsn_runtime *rt) { RT_CHECK(rt); return rt->rt.dev.sync(); }
int tsn_runtime_alloc_stats(tsn_runtime *rt, size_t *count, size_t *bytes) {
    RT_CHECK(rt);
    if (count) *count = rt->rt.dev.owned_count();
    if (bytes) *bytes = rt->rt.dev.owned_bytes();
    return TSN_OK;
}

int tsn_gemm(tsn_runtime *rt, int wdtype, const void *W, const void *X, int xdtype, void *Y, int ydtype,
             const float *bias, uint32_t M, uint32_t N, uint32_t K, uint32_t ldx, uint32_t ldw, uint32_t ldy) {
    RT_CHECK(rt);
    return rt->rt.gemm(wdtype, W, X, xdtype, Y, ydtype, bias, tsn::GemmParams{M, N, K, ldx, ldw, ldy});
}
int tsn_gemm_noalloc(tsn_runtime *rt, int wdtype, const void *W, const void *X, int xdtype, void *Y, int ydtype,
                     const float *bias, uint32_t M, uint32_t N, uint32_t K, uint32_t ldx, uint32_t ldw, uint32_t ldy) {
    RT_CHECK(rt);
    return tsn::gemm_noalloc(rt->rt, wdtype, W, X, xdtype, Y, ydtype, bias, tsn::GemmParams{M, N, K, ldx, ldw, ldy});
}
size_t tsn_gemm_noalloc_max_elems(void) { return tsn::noalloc_scratch_bytes() / 4; }
int tsn_gemv(tsn_runtime *rt, const void *W, int wdtype, const float *x, float *y, const float *bias, uint32_t N,
             uint32_t K, uint32_t ldw) {
    RT_CHECK(rt);
    return rt->rt.gemv(W, x, y, bias, N, K, ldw, wdtype);
}
size_t tsn_conv1d_prepared_bytes(int wdtype, uint32_t OC, uint32_t IC, uint32_t K) {
    if (wdtype != TSN_F32 && wdtype != TSN_F16 && wdtype != TSN_BF16) return 0;
    return (size_t)OC * (size_t)tsn::conv_prep_cols(wdtype, (int)IC, (int)K) * sizeof(tsn::half_t);
}
int tsn_conv1d_prepare(tsn_runtime *rt, const void *W, int wdtype, void *Wp, uint32_t OC, uint32_t IC, uint32_t K) {
    RT_CHECK(rt);
    return rt->rt.conv_prepare(W, wdtype, Wp, OC, IC, K);
}
int tsn_conv1d(tsn_runtime *rt, int wdtype, const void *Wp, const float *bias, const float *x, float *y, uint32_t T,
               uint32_t OL, uint32_t IC, uint32_t OC, uint32_t K, uint32_t stride, uint32_t pad, uint32_t dil,
               int convt) {
    RT_CHECK(rt);
    return rt->rt.conv(wdtype, Wp, bias, x, y, T, OL, IC, OC, K, stride, pad, dil, convt ? 1u : 0u);
}
int tsn_silu(tsn_runtime *rt, float *x, size_t n) { RT_CHECK(rt); return rt->rt.silu(x, n); }
int tsn_copy(tsn_runtime *rt, const float *x, float *y, size_t n) { RT_CHECK(rt); return rt->rt.copy(x, y, n); }
int tsn_swiglu(tsn_runtime *rt, const float *a, const float *b, float *y, size_t n) { RT_CHECK(rt); return rt->rt.swiglu(a, b, y, n); }
int tsn_add(tsn_runtime *rt, const float *a, const float *b, float *y, size_t n) { RT_CHECK(rt); return rt->rt.add_(a, b, y, n); }
int tsn_add_bcast_col(tsn_runtime *rt, const float *x, const float *v, float *y, uint32_t S, uint32_t H) {
    RT_CHECK(rt);
    return rt->rt.add_bcast_col(x, v, y, S, H);
}
int tsn_cfg_euler(tsn_runtime *rt, const float *fc, const float *fu, float *x, size_t n, float cfg, float dt) {
    RT_CHECK(rt);
    return rt->rt.cfg_euler(fc, fu, x, n, cfg, dt);
}
int tsn_geglu(tsn_runtime *rt, const float *a, const float *b, float *y, size_t n) { RT_CHECK(rt); return rt->rt.geglu(a, b, y, n); }
int tsn_gelu_quick(tsn_runtime *rt, float *x, size_t n) { RT_CHECK(rt); return rt->rt.gelu_quick(x, n); }
int tsn_ln_plain(tsn_runtime *rt, const float *x, float *y, uint32_t S, uint32_t H, float eps) {
    RT_CHECK(rt);
    return rt->rt.ln_plain(x, y, S, H, eps);
}
int tsn_ln_wb(tsn_runtime *rt, const float *x, float *y, const float *w, const float *b, uint32_t S, uint32_t H,
              float eps) {
    RT_CHECK(rt);
    return rt->rt.ln_wb(x, y, w, b, S, H, eps);
}
int tsn_rms_w(tsn_runtime *rt, const float *x, float *y, const float *w, uint32_t S, uint32_t H, float eps) {
    RT_CHECK(rt);
    return rt->rt.rms_w(x, y, w, S, H, eps);
}
int tsn_mean_cols(tsn_runtime *rt, const float *x, float *y, uint32_t S, uint32_t H) {
    RT_CHECK(rt);
    return rt->rt.mean_cols(x, y, S, H);
}
int tsn_qkv_split3(tsn_runtime *rt, const float *src, float *dst, uint32_t rows, uint32_t H, uint32_t row_off) {
    RT_CHECK(rt);
    return rt->rt.qkv_split3(src, dst, rows, H, row_off);
}
int tsn_adaln_ln(tsn_runtime *rt, const float *x, const float *mod, void *y, int ydtype, uint32_t rows, uint32_t H,
                 uint32_t per_row, uint32_t chunks, uint32_t base, float eps) {
    RT_CHECK(rt);
    return rt->rt.adaln_ln(x, mod, y, ydtype, rows, H, per_row, chunks, base, eps);
}
int tsn_gate_add(tsn_runtime *rt, const float *x, const float *f, const float *mod, float *y, uint32_t rows, uint32_t H,
                 uint32_t per_row, uint32_t chunks, uint32_t gate_idx) {
    RT_CHECK(rt);
    return rt->rt.gate_add(x, f, mod, y, rows, H, per_row, chunks, gate_idx);
}
int tsn_rms_head(tsn_runtime *rt, float *x, const float *w, uint32_t rows, uint32_t nh, uint32_t ld, uint32_t hd,
                 uint32_t col_off, uint32_t row_off, float eps) {
    RT_CHECK(rt);
    return rt->rt.rms_head(x, w, rows, nh, ld, hd, col_off, row_off, eps);
}
int tsn_rope_pairs(tsn_runtime *rt, float *x, const int32_t *pos, uint32_t rows, uint32_t nh, uint32_t ld, uint32_t hd,
                   uint32_t col_off, uint32_t row_off, float fscale, float base) {
    RT_CHECK(rt);
    return rt->rt.rope_pairs(x, pos, rows, nh, ld, hd, col_off, row_off, fscale, base);
}
int tsn_attention(tsn_runtime *rt, const float *qkv, float *out, uint32_t S, uint32_t nh, uint32_t hd, uint32_t ld,
                  uint32_t ldo, uint32_t q_off, uint32_t k_off, uint32_t v_off, uint32_t o_off, float scale) {
    RT_CHECK(rt);
    return rt->rt.attention(qkv, out, S, nh, hd, ld, ldo, q_off, k_off, v_off, o_off, scale);
}

int tsn_probe_peaks(tsn_runtime *rt, double *mfma_tflops, double *hbm_gbs) {
    RT_CHECK(rt);
    return rt->rt.probe_peaks(mfma_tflops, hbm_gbs);
}

int tsn_dit_default_spec(int workload, tsn_dit_spec *out) {
    if (!out || workload < 0 || workload > 4) { tsn::set_error("default_spec: workload must be 0..4"); return TSN_ERR_ARG; }
    tsn_dit_spec s;
    memset(&s, 0, sizeof s);
    s.B = workload == 4 ? 16 : 2;
    s.La = workload == 3 ? 960 : 256;
    s.Lt = 141;
    s.H = 1024; s.NH = 16; s.HD = 64; s.F = 4096;
    s.latent = 64; s.temb_dim = 256;
    s.n_joint = 7; s.n_fused = 14;
    s.audio_ffn_conv = 1;
    s.rope_theta = 10000.0f; s.t_max_period = 1.0f; s.ln_eps = 1e-5f; s.rms_eps = 1e-6f;
    *out = s;
    return TSN_OK;
}

int tsn_dit_manifest_count(const tsn_dit_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    return (int)tsn::dit_manifest(to_spec(spec)).size();
}
int tsn_dit_manifest_entry(const tsn_dit_spec *spec, int idx, char *name, int name_cap, int64_t *numel, int64_t *offset) {
    if (!spec) { tsn::set_error("null spec"); return TSN_ERR_ARG; }
    const auto m = tsn::dit_manifest(to_spec(spec));
    if (idx < 0 || idx >= (int)m.size()) { tsn::set_error("manifest index out of range"); return TSN_ERR_ARG; }
    if (name && name_cap > 0) snprintf(name, (size_t)name_cap, "%s", m[idx].name.c_str());
    if (numel) *numel = m[idx].numel;
    if (offset) *offset = m[idx].offset;
    return TSN_OK;
}
int64_t tsn_dit_manifest_total(const tsn_dit_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    const auto m = tsn::dit_manifest(to_spec(spec));
    return m.back().offset + m.back().numel;
}

int tsn_dit_create(tsn_runtime *rt, const tsn_dit_spec *spec, tsn_dit **out) {
    RT_CHECK(rt);
    if (!spec || !out) { tsn::set_error("null spec or out pointer"); return TSN_ERR_ARG; }
    *out = nullptr;
    tsn_dit *d = new (std::nothrow) tsn_dit();
    if (!d) { tsn::set_error("out of host memory"); return TSN_ERR_OOM; }
    const int rc = d->m.create(&rt->rt, to_spec(spec));
    if (rc != TSN_OK) { delete d; return rc; }
    *out = d;
    return TSN_OK;
}
int tsn_dit_destroy(tsn_dit *dit) { delete dit; return TSN_OK; }
int tsn_dit_upload_weights(tsn_dit *dit, const uint16_t *w, size_t numel) {
    if (!dit) { tsn::set_error("null dit handle"); return TSN_ERR_ARG; }
    return dit->m.upload_weights(w, numel);
}
int tsn_dit_forward(tsn_dit *dit, const float *z, float t, const float *text, const float *pooled, float *v) {
    if (!dit) { tsn::set_error("null dit handle"); return TSN_ERR_ARG; }
    tsn::DitModel &m = dit->m;
    std::vector<float> th((size_t)m.s.B, t);
    TSN_TRY(m.rt->dev.upload(m.t_dev, th.data(), th.size() * 4));
    return m.enqueue_forward(z, m.t_dev, text, pooled, v, nullptr);
}
int tsn_dit_forward_ex(tsn_dit *dit, const float *z, const float *t, const float *text, const float *pooled, float *v,
                       float *taps) {
    if (!dit) { tsn::set_error("null dit handle"); return TSN_ERR_ARG; }
    return dit->m.enqueue_forward(z, t, text, pooled, v, taps);
}
int tsn_dit_joint_block(tsn_dit *dit, int block, float *X, const float *g) {
    if (!dit) { tsn::set_error("null dit handle"); return TSN_ERR_ARG; }
    return dit->m.enqueue_joint_block(block, X, g);
}
int tsn_dit_fused_block(tsn_dit *dit, int block, float *X, const float *g) {
    if (!dit) { tsn::set_error("null dit handle"); return TSN_ERR_ARG; }
    return dit->m.enqueue_fused_block(block, X, g);
}
int tsn_dit_sample(tsn_dit *dit, float *x, const float *text, const float *pooled, int steps, float cfg) {
    if (!dit) { tsn::set_error("null dit handle"); return TSN_ERR_ARG; }
    TSN_TRY(dit->m.prepare_sample(steps));
    return dit->m.enqueue_sample(x, text, pooled, steps, cfg);
}
int tsn_dit_capture_forward(tsn_dit *dit, const float *z, const float *t, const float *text, const float *pooled, float *v) {
    if (!dit) { tsn::set_error("null dit handle"); return TSN_ERR_ARG; }
    return dit->m.capture_forward(z, t, text, pooled, v);
}
int tsn_dit_capture_sample(tsn_dit *dit, float *x, const float *text, const float *pooled, int steps, float cfg) {
    if (!dit) { tsn::set_error("null dit handle"); return TSN_ERR_ARG; }
    return dit->m.capture_sample(x, text, pooled, steps, cfg);
}
int tsn_dit_replay(tsn_dit *dit) {
    if (!dit) { tsn::set_error("null dit handle"); return TSN_ERR_ARG; }
    return dit->m.replay();
}

int tsn_dit_profile_forward(tsn_dit *dit, const float *z, const float *t, const float *text, const float *pooled,
                            float *v, tsn_kernel_stat *stats, int cap, int *n_stats) {
    if (!dit || !stats || !n_stats || cap <= 0) { tsn::set_error("profile: null argument"); return TSN_ERR_ARG; }
    std::vector<tsn::KernelStat> ks;
    const int rc = dit->m.profile_forward(z, t, text, pooled, v, ks);
    if (rc != TSN_OK) return rc;
    return copy_stats(ks, stats, cap, n_stats);
}

/* ---------------- reference graph ---------------- */
#define REF_CHECK(d)                                                              \
    do {                                                                          \
        if (!(d)) { tsn::set_error("null refdit handle"); return TSN_ERR_ARG; }   \
    } while (0)

int tsn_refdit_spec_for_duration(int dur_s, int B, tsn_refdit_spec *out) {
    if (!out || dur_s <= 0) { tsn::set_error("refdit spec: null out pointer or non-positive duration"); return TSN_ERR_ARG; }
    const tsn::RefDitSpec s = tsn::refdit_spec_for_duration(dur_s, B);
    out->B = s.B; out->T = s.T; out->C = s.C; out->TS = s.TS; out->H = s.H; out->NH = s.NH; out->HD = s.HD;
    out->F = s.F; out->latent = s.latent; out->n_joint = s.n_joint; out->n_fused = s.n_fused;
    out->rope_theta = s.rope_theta; out->t_max_period = s.t_max_period; out->ln_eps = s.ln_eps; out->rms_eps = s.rms_eps;
    return tsn::refdit_spec_check(s);
}
int tsn_refdit_manifest_count(const tsn_refdit_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    return (int)tsn::refdit_manifest(to_ref_spec(spec)).size();
}
int tsn_refdit_manifest_entry(const tsn_refdit_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                              int64_t *offset) {
    if (!spec) { tsn::set_error("null spec"); return TSN_ERR_ARG; }
    const auto m = tsn::refdit_manifest(to_ref_spec(spec));
    if (idx < 0 || idx >= (int)m.size()) { tsn::set_error("manifest index out of range"); return TSN_ERR_ARG; }
    if (name && name_cap > 0) snprintf(name, (size_t)name_cap, "%s", m[idx].name.c_str());
    if (numel) *numel = m[idx].numel;
    if (offset) *offset = m[idx].offset;
    return TSN_OK;
}
int64_t tsn_refdit_manifest_total(const tsn_refdit_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    const auto m = tsn::refdit_manifest(to_ref_spec(spec));
    return m.back().offset + m.back().numel;
}
int tsn_refdit_create(tsn_runtime *rt, const tsn_refdit_spec *spec, tsn_refdit **out) {
    RT_CHECK(rt);
    if (!spec || !out) { tsn::set_error("null spec or out pointer"); return TSN_ERR_ARG; }
    *out = nullptr;
    tsn_refdit *d = new (std::nothrow) tsn_refdit();
    if (!d) { tsn::set_error("out of host memory"); return TSN_ERR_OOM; }
    const int rc = d->m.create(&rt->rt, to_ref_spec(spec));
    if (rc != TSN_OK) { delete d; return rc; }
    *out = d;
    return TSN_OK;
}
int tsn_refdit_destroy(tsn_refdit *d) { delete d; return TSN_OK; }
int tsn_refdit_upload_weights(tsn_refdit *d, const uint16_t *w, size_t numel) {
    REF_CHECK(d);
    return d->m.upload_weights(w, numel);
}
int tsn_refdit_upload_weights_f32(tsn_refdit *d, const float *w, size_t numel) {
    REF_CHECK(d);
    return d->m.upload_weights_f32(w, numel);
}
int tsn_refdit_load_gguf(tsn_refdit *d, const char *path) {
    REF_CHECK(d);
    if (!path) { tsn::set_error("null path"); return TSN_ERR_ARG; }
    return d->m.load_gguf(path);
}
int tsn_refdit_spec_from_gguf(const char *path, int B, int T, int C, int TS, tsn_refdit_spec *out) {
    if (!path || !out) { tsn::set_error("null path or spec"); return TSN_ERR_ARG; }
    tsn::RefDitSpec s;
    TSN_TRY(tsn::refdit_spec_from_gguf(path, B, T, C, TS, &s));
    out->B = s.B; out->T = s.T; out->C = s.C; out->TS = s.TS; out->H = s.H; out->NH = s.NH; out->HD = s.HD;
    out->F = s.F; out->latent = s.latent; out->n_joint = s.n_joint; out->n_fused = s.n_fused;
    out->rope_theta = s.rope_theta; out->t_max_period = s.t_max_period; out->ln_eps = s.ln_eps; out->rms_eps = s.rms_eps;
    return TSN_OK;
}

/* ---------------- conditioning prep ---------------- */
#define COND_CHECK(d)                                                             \
    do {                                                                          \
        if (!(d)) { tsn::set_error("null refcond handle"); return TSN_ERR_ARG; }  \
    } while (0)

int tsn_refcond_spec_for_duration(int dur_s, tsn_refcond_spec *out) {
    if (!out || dur_s <= 0) { tsn::set_error("refcond spec: null out pointer or non-positive duration"); return TSN_ERR_ARG; }
    from_cond_spec(tsn::refcond_spec_for_duration(dur_s), out);
    return TSN_OK;
}
int tsn_refcond_spec_from_gguf(const char *path, int T, int C, int sync_S, int TS, tsn_refcond_spec *out) {
    if (!path || !out) { tsn::set_error("null path or spec"); return TSN_ERR_ARG; }
    tsn::RefCondSpec s;
    TSN_TRY(tsn::refcond_spec_from_gguf(path, T, C, sync_S, TS, &s));
    from_cond_spec(s, out);
    return TSN_OK;
}
int tsn_refcond_manifest_count(const tsn_refcond_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    return (int)tsn::refcond_manifest(to_cond_spec(spec)).size();
}
int tsn_refcond_manifest_entry(const tsn_refcond_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                               int64_t *offset) {
    if (!spec) { tsn::set_error("null spec"); return TSN_ERR_ARG; }
    const auto m = tsn::refcond_manifest(to_cond_spec(spec));
    if (idx < 0 || idx >= (int)m.size()) { tsn::set_error("manifest index out of range"); return TSN_ERR_ARG; }
    if (name && name_cap > 0) snprintf(name, (size_t)name_cap, "%s", m[idx].name.c_str());
    if (numel) *numel = m[idx].numel;
    if (offset) *offset = m[idx].offset;
    return TSN_OK;
}
int64_t tsn_refcond_manifest_total(const tsn_refcond_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    const auto m = tsn::refcond_manifest(to_cond_spec(spec));
    return m.back().offset + m.back().numel;
}
int tsn_refcond_create(tsn_runtime *rt, const tsn_refcond_spec *spec, tsn_refcond **out) {
    RT_CHECK(rt);
    if (!spec || !out) { tsn::set_error("null spec or out pointer"); return TSN_ERR_ARG; }
    *out = nullptr;
    tsn_refcond *d = new (std::nothrow) tsn_refcond();
    if (!d) { tsn::set_error("out of host memory"); return TSN_ERR_OOM; }
    const int rc = d->m.create(&rt->rt, to_cond_spec(spec));
    if (rc != TSN_OK) { delete d; return rc; }
    *out = d;
    return TSN_OK;
}
int tsn_refcond_destroy(tsn_refcond *d) { delete d; return TSN_OK; }
int tsn_refcond_upload_weights(tsn_refcond *d, const uint16_t *w, size_t numel) {
    COND_CHECK(d);
    return d->m.upload_weights(w, numel);
}
int tsn_refcond_upload_weights_f32(tsn_refcond *d, const float *w, size_t numel) {
    COND_CHECK(d);
    return d->m.upload_weights_f32(w, numel);
}
int tsn_refcond_load_gguf(tsn_refcond *d, const char *path) {
    COND_CHECK(d);
    if (!path) { tsn::set_error("null path"); return TSN_ERR_ARG; }
    return d->m.load_gguf(path);
}
int tsn_refcond_prep_conditioning(tsn_refcond *d, const float *clip_f, const float *sync_f, float *clip_pp,
                                  float *sync_gather, float *clip_fc) {
    COND_CHECK(d);
    return d->m.enqueue_prep_conditioning(clip_f, sync_f, clip_pp, sync_gather, clip_fc);
}
int tsn_refcond_prep_text_arm(tsn_refcond *d, const float *text_cat, const float *gtext, const float *clip_fc,
                              float *text_pp, float *gcmlp) {
    COND_CHECK(d);
    return d->m.enqueue_prep_text_arm(text_cat, gtext, clip_fc, text_pp, gcmlp);
}

/* ---------------- VAE decoder ---------------- */
#define VAE_CHECK(d)                                                          \
    do {                                                                      \
        if (!(d)) { tsn::set_error("null vae handle"); return TSN_ERR_ARG; }  \
    } while (0)

int tsn_vae_spec_for_duration(int dur_s, tsn_vae_spec *out) {
    if (!out || dur_s <= 0) { tsn::set_error("vae spec: null out pointer or non-positive duration"); return TSN_ERR_ARG; }
    from_vae_spec(tsn::vae_spec_for_duration(dur_s), out);
    return TSN_OK;
}
int tsn_vae_spec_from_gguf(const char *path, int T, tsn_vae_spec *out) {
    if (!path || !out) { tsn::set_error("null path or spec"); return TSN_ERR_ARG; }
    tsn::VaeSpec s;
    TSN_TRY(tsn::vae_spec_from_gguf(path, T, &s));
    from_vae_spec(s, out);
    return TSN_OK;
}
int64_t tsn_vae_audio_len(const tsn_vae_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    return tsn::vae_audio_len(to_vae_spec(spec));
}
int tsn_vae_manifest_count(const tsn_vae_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    return (int)tsn::vae_manifest(to_vae_spec(spec)).size();
}
int tsn_vae_manifest_entry(const tsn_vae_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                           int64_t *offset) {
    if (!spec) { tsn::set_error("null spec"); return TSN_ERR_ARG; }
    const auto m = tsn::vae_manifest(to_vae_spec(spec));
    if (idx < 0 || idx >= (int)m.size()) { tsn::set_error("manifest index out of range"); return TSN_ERR_ARG; }
    if (name && name_cap > 0) snprintf(name, (size_t)name_cap, "%s", m[idx].name.c_str());
    if (numel) *numel = m[idx].numel;
    if (offset) *offset = m[idx].offset;
    return TSN_OK;
}
int64_t tsn_vae_manifest_total(const tsn_vae_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    const auto m = tsn::vae_manifest(to_vae_spec(spec));
    return m.back().offset + m.back().numel;
}
int tsn_vae_create(tsn_runtime *rt, const tsn_vae_spec *spec, tsn_vae **out) {
    RT_CHECK(rt);
    if (!spec || !out) { tsn::set_error("null spec or out pointer"); return TSN_ERR_ARG; }
    *out = nullptr;
    tsn_vae *d = new (std::nothrow) tsn_vae();
    if (!d) { tsn::set_error("out of host memory"); return TSN_ERR_OOM; }
    const int rc = d->m.create(&rt->rt, to_vae_spec(spec));
    if (rc != TSN_OK) { delete d; return rc; }
    *out = d;
    return TSN_OK;
}
int tsn_vae_destroy(tsn_vae *d) { delete d; return TSN_OK; }
int tsn_vae_upload_weights(tsn_vae *d, const float *w, size_t numel) {
    VAE_CHECK(d);
    return d->m.upload_weights(w, numel);
}
int tsn_vae_load_gguf(tsn_vae *d, const char *path) {
    VAE_CHECK(d);
    if (!path) { tsn::set_error("null path"); return TSN_ERR_ARG; }
    return d->m.load_gguf(path);
}
int tsn_vae_decode(tsn_vae *d, const float *latent, float *audio) {
    VAE_CHECK(d);
    return d->m.enqueue_decode(latent, audio);
}
int tsn_vae_capture_decode(tsn_vae *d, const float *latent, float *audio) {
    VAE_CHECK(d);
    return d->m.capture([&] { return d->m.enqueue_decode(latent, audio); });
}
int tsn_vae_replay(tsn_vae *d) {
    VAE_CHECK(d);
    return d->m.replay();
}
int tsn_vae_profile_decode(tsn_vae *d, const float *latent, float *audio, tsn_kernel_stat *stats, int cap,
                           int *n_stats) {
    if (!d || !stats || !n_stats || cap <= 0) { tsn::set_error("profile: null argument"); return TSN_ERR_ARG; }
    std::vector<tsn::KernelStat> ks;
    const int rc = d->m.profile([&] { return d->m.enqueue_decode(latent, audio); }, ks);
    if (rc != TSN_OK) return rc;
    return copy_stats(ks, stats, cap, n_stats);
}

/* ---------------- text encoders ---------------- */
#define ENC_CHECK(d, what)                                                              \
    do {                                                                                \
        if (!(d)) { tsn::set_error("null " what " handle"); return TSN_ERR_ARG; }       \
    } while (0)

int tsn_clip_spec_default(tsn_clip_spec *out) {
    if (!out) { tsn::set_error("null spec"); return TSN_ERR_ARG; }
    from_clip_spec(tsn::clip_spec_default(), out);
    return TSN_OK;
}
int tsn_clip_spec_from_gguf(const char *path, tsn_clip_spec *out) {
    if (!path || !out) { tsn::set_error("null path or spec"); return TSN_ERR_ARG; }
    tsn::ClipSpec s;
    TSN_TRY(tsn::clip_spec_from_gguf(path, &s));
    from_clip_spec(s, out);
    return TSN_OK;
}
int tsn_clip_manifest_count(const tsn_clip_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    return (int)tsn::clip_manifest(to_clip_spec(spec)).size();
}
int tsn_clip_manifest_entry(const tsn_clip_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                            int64_t *offset) {
    if (!spec) { tsn::set_error("null spec"); return TSN_ERR_ARG; }
    return manifest_entry(tsn::clip_manifest(to_clip_spec(spec)), idx, name, name_cap, numel, offset);
}
int64_t tsn_clip_manifest_total(const tsn_clip_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    const auto m = tsn::clip_manifest(to_clip_spec(spec));
    return m.back().offset + m.back().numel;
}
int tsn_clip_create(tsn_runtime *rt, const tsn_clip_spec *spec, tsn_clip **out) {
    RT_CHECK(rt);
    if (!spec || !out) { tsn::set_error("null spec or out pointer"); return TSN_ERR_ARG; }
    *out = nullptr;
    tsn_clip *d = new (std::nothrow) tsn_clip();
    if (!d) { tsn::set_error("out of host memory"); return TSN_ERR_OOM; }
    const int rc = d->m.create(&rt->rt, to_clip_spec(spec));
    if (rc != TSN_OK) { delete d; return rc; }
    *out = d;
    return TSN_OK;
}
int tsn_clip_destroy(tsn_clip *d) { delete d; return TSN_OK; }
int tsn_clip_upload_weights(tsn_clip *d, const float *w, size_t numel) {
    ENC_CHECK(d, "clip");
    return d->m.upload_weights(w, numel);
}
int tsn_clip_load_gguf(tsn_clip *d, const char *path) {
    ENC_CHECK(d, "clip");
    if (!path) { tsn::set_error("null path"); return TSN_ERR_ARG; }
    return d->m.load_gguf(path);
}
int tsn_clip_encode(tsn_clip *d, const int32_t *ids, float *per_token, float *global) {
    ENC_CHECK(d, "clip");
    return d->m.encode(ids, per_token, global);
}
int tsn_clip_profile_encode(tsn_clip *d, const int32_t *ids, float *per_token, float *global, tsn_kernel_stat *stats,
                            int cap, int *n_stats) {
    if (!d || !stats || !n_stats || cap <= 0) { tsn::set_error("profile: null argument"); return TSN_ERR_ARG; }
    std::vector<tsn::KernelStat> ks;
    const int rc = d->m.profile([&] { return d->m.encode(ids, per_token, global); }, ks);
    if (rc != TSN_OK) return rc;
    return copy_stats(ks, stats, cap, n_stats);
}
int tsn_t5_spec_default(tsn_t5_spec *out) {
    if (!out) { tsn::set_error("null spec"); return TSN_ERR_ARG; }
    from_t5_spec(tsn::t5_spec_default(), out);
    return TSN_OK;
}
int tsn_t5_spec_from_gguf(const char *path, tsn_t5_spec *out) {
    if (!path || !out) { tsn::set_error("null path or spec"); return TSN_ERR_ARG; }
    tsn::T5Spec s;
    TSN_TRY(tsn::t5_spec_from_gguf(path, &s));
    from_t5_spec(s, out);
    return TSN_OK;
}
int tsn_t5_manifest_count(const tsn_t5_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    return (int)tsn::t5_manifest(to_t5_spec(spec)).size();
}
int tsn_t5_manifest_entry(const tsn_t5_spec *spec, int idx, char *name, int name_cap, int64_t *numel,
                          int64_t *offset) {
    if (!spec) { tsn::set_error("null spec"); return TSN_ERR_ARG; }
    return manifest_entry(tsn::t5_manifest(to_t5_spec(spec)), idx, name, name_cap, numel, offset);
}
int64_t tsn_t5_manifest_total(const tsn_t5_spec *spec) {
    if (!spec) { tsn::set_error("null spec"); return -1; }
    const auto m = tsn::t5_manifest(to_t5_spec(spec));
    return m.back().offset + m.back().numel;
}
int tsn_t5_create(tsn_runtime *rt, const tsn_t5_spec *spec, tsn_t5 **out) {
    RT_CHECK(rt);
    if (!spec || !out) { tsn::set_error("null spec or out pointer"); return TSN_ERR_ARG; }
    *out = nullptr;
    tsn_t5 *d = new (std::nothrow) tsn_t5();
    if (!d) { tsn::set_error("out of host memory"); return TSN_ERR_OOM; }
    const int rc = d->m.create(&rt->rt, to_t5_spec(spec));
    if (rc != TSN_OK) { delete d; return rc; }
    *out = d;
    return TSN_OK;
}
int tsn_t5_destroy(tsn_t5 *d) { delete d; return TSN_OK; }
int tsn_t5_upload_weights(tsn_t5 *d, const float *w, size_t numel) {
    ENC_CHECK(d, "t5");
    return d->m.upload_weights(w, numel);
}
int tsn_t5_load_gguf(tsn_t5 *d, const char *path) {
    ENC_CHECK(d, "t5");
    if (!path) { tsn::set_error("null path"); return TSN_ERR_ARG; }
    return d->m.load_gguf(path);
}
int tsn_t5_encode(tsn_t5 *d, const int32_t *ids, float *out) {
    ENC_CHECK(d, "t5");
    return d->m.encode(ids, out);
}
int tsn_t5_profile_encode(tsn_t5 *d, const int32_t *ids, float *out, tsn_kernel_stat *stats, int cap, int *n_stats) {
    if (!d || !stats || !n_stats || cap <= 0) { tsn::set_error("profile: null argument"); return TSN_ERR_ARG; }
    std::vector<tsn::KernelStat> ks;
    const int rc = d->m.profile([&] { return d->m.encode(ids, out); }, ks);
    if (rc != TSN_OK) return rc;
    return copy_stats(ks, stats, cap, n_stats);
}
int tsn_t5_bucket(int rel, int n_bucket, int max_dist) {
    if (n_bucket < 4 || n_bucket % 4 || max_dist <= n_bucket / 4) {
        tsn::set_error("t5 bucket: n_bucket a multiple of 4, max_dist past the exact range");
        return -1;
    }
    return tsn::t5_bucket(rel, n_bucket, max_dist);
}

/* ---------------- tokenizers ---------------- */
int tsn_clip_tokenizer_load(const char *path, tsn_clip_tokenizer **out) {
    if (!path || !out) { tsn::set_error("null path or out pointer"); return TSN_ERR_ARG; }
    *out = nullptr;
    tsn_clip_tokenizer *t = new (std::nothrow) tsn_clip_tokenizer();
    if (!t) { tsn::set_error("out of host memory"); return TSN_ERR_OOM; }
    const int rc = t->t.load(path);
    if (rc != TSN_OK) { delete t; return rc; }
    *out = t;
    return TSN_OK;
}
int tsn_clip_tokenizer_destroy(tsn_clip_tokenizer *t) { delete t; return TSN_OK; }
int tsn_clip_tokenizer_encode(const tsn_clip_tokenizer *t, const char *text, int ctx, int32_t *ids) {
    if (!t || !text || !ids || ctx < 2) { tsn::set_error("clip tokenizer: null argument or ctx < 2"); return TSN_ERR_ARG; }
    const auto v = t->t.encode(text, ctx);
    memcpy(ids, v.data(), v.size() * sizeof(int32_t));
    return TSN_OK;
}
int tsn_t5_tokenizer_load(const char *path, tsn_t5_tokenizer **out) {
    if (!path || !out) { tsn::set_error("null path or out pointer"); return TSN_ERR_ARG; }
    *out = nullptr;
    tsn_t5_tokenizer *t = new (std::nothrow) tsn_t5_tokenizer();
    if (!t) { tsn::set_error("out of host memory"); return TSN_ERR_OOM; }
    const int rc = t->t.load(path);
    if (rc != TSN_OK) { delete t; return rc; }
    *out = t;
    return TSN_OK;
}
int tsn_t5_tokenizer_destroy(tsn_t5_tokenizer *t) { delete t; return TSN_OK; }
int tsn_t5_tokenizer_encode(const tsn_t5_tokenizer *t, const char *text, int ctx, int pad, int32_t *ids, int *n_ids) {
    if (!t || !text || !ids || !n_ids || ctx < 1) { tsn::set_error("t5 tokenizer: null argument or ctx < 1"); return TSN_ERR_ARG; }
    const auto v = t->t.encode(text, ctx, pad != 0);
    memcpy(ids, v.data(), v.size() * sizeof(int32_t));
    *n_ids = (int)v.size();
    return TSN_OK;
}

/* ---------------- GGUF reader ---------------- */
int tsn_gguf_open(const char *path, tsn_gguf **out) {
    if (!path || !out) { tsn::set_error("null path or out pointer"); return TSN_ERR_ARG; }
    *out = nullptr;
    tsn_gguf *g = new (std::nothrow) tsn_gguf();
    if (!g) { tsn::set_error("out of host memory"); return TSN_ERR_OOM; }
    const int rc = g->r.open(path);
    if (rc != TSN_OK) { delete g; return rc; }
    *out = g;
    return TSN_OK;
}
int tsn_gguf_close(tsn_gguf *g) { delete g; return TSN_OK; }
int tsn_gguf_tensor_count(const tsn_gguf *g) {
    if (!g) { tsn::set_error("null gguf handle"); return -1; }
    return (int)g->r.tensors().size();
}
int tsn_gguf_tensor_info(const tsn_gguf *g, int idx, char *name, int name_cap, uint32_t *type, uint32_t *n_dims,
                         uint64_t *ne4) {
    if (!g) { tsn::set_error("null gguf handle"); return TSN_ERR_ARG; }
    const auto &v = g->r.tensors();
    if (idx < 0 || idx >= (int)v.size()) { tsn::set_error("tensor index out of range"); return TSN_ERR_ARG; }
    const tsn::GgufTensorInfo &t = v[idx];
    if (name && name_cap > 0) snprintf(name, (size_t)name_cap, "%s", t.name.c_str());
    if (type) *type = t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (ne4)
        for (int d = 0; d < 4; ++d) ne4[d] = t.ne[d];
    return TSN_OK;
}
int tsn_gguf_tensor_to_f32(const tsn_gguf *g, const char *name, float *out, size_t cap) {
    if (!g || !name || !out) { tsn::set_error("null argument"); return TSN_ERR_ARG; }
    const tsn::GgufTensorInfo *t = g->r.find(name);
    if (!t) { tsn::set_error(std::string("gguf: no tensor ") + name); return TSN_ERR_ARG; }
    if (cap < t->numel()) { tsn::set_error("gguf: output too small"); return TSN_ERR_ARG; }
    return g->r.to_f32(*t, out);
}
int64_t tsn_gguf_get_i64(const tsn_gguf *g, const char *key, int64_t def) {
    return g && key ? g->r.get_i64(key, def) : def;
}
double tsn_gguf_get_f64(const tsn_gguf *g, const char *key, double def) {
    return g && key ? g->r.get_f64(key, def) : def;
}

int tsn_refdit_forward(tsn_refdit *d, const float *x, float t, const float *clip_pp, const float *text_pp,
                       const float *gcmlp, const float *sync_gather, float *flow) {
    REF_CHECK(d);
    tsn::RefDitModel &m = d->m;
    std::vector<float> th((size_t)m.s.B, t);
    TSN_TRY(m.rt->dev.upload(m.t_dev, th.data(), th.size() * 4));
    return m.enqueue_forward(x, m.t_dev, clip_pp, text_pp, gcmlp, sync_gather, flow, nullptr);
}
int tsn_refdit_forward_ex(tsn_refdit *d, const float *x, const float *t, const float *clip_pp, const float *text_pp,
                          const float *gcmlp, const float *sync_gather, float *flow, float *taps) {
    REF_CHECK(d);
    return d->m.enqueue_forward(x, t, clip_pp, text_pp, gcmlp, sync_gather, flow, taps);
}
int tsn_refdit_sample(tsn_refdit *d, float *x, const float *clip_pp, const float *text_pp, const float *gcmlp,
                      const float *sync_gather, int steps, float cfg) {
    REF_CHECK(d);
    TSN_TRY(d->m.prepare_sample(steps));
    return d->m.enqueue_sample(x, clip_pp, text_pp, gcmlp, sync_gather, steps, cfg);
}
int tsn_refdit_capture_forward(tsn_refdit *d, const float *x, const float *t, const float *clip_pp,
                               const float *text_pp, const float *gcmlp, const float *sync_gather, float *flow) {
    REF_CHECK(d);
    return d->m.capture_forward(x, t, clip_pp, text_pp, gcmlp, sync_gather, flow);
}
int tsn_refdit_capture_sample(tsn_refdit *d, float *x, const float *clip_pp, const float *text_pp, const float *gcmlp,
                              const float *sync_gather, int steps, float cfg) {
    REF_CHECK(d);
    return d->m.capture_sample(x, clip_pp, text_pp, gcmlp, sync_gather, steps, cfg);
}
int tsn_refdit_replay(tsn_refdit *d) {
    REF_CHECK(d);
    return d->m.replay();
}
int tsn_refdit_profile_forward(tsn_refdit *d, const float *x, const float *t, const float *clip_pp,
                               const float *text_pp, const float *gcmlp, const float *sync_gather, float *flow,
                               tsn_kernel_stat *stats, int cap, int *n_stats) {
    if (!d || !stats || !n_stats || cap <= 0) { tsn::set_error("profile: null argument"); return TSN_ERR_ARG; }
    std::vector<tsn::KernelStat> ks;
    const int rc = d->m.profile_forward(x, t, clip_pp, text_pp, gcmlp, sync_gather, flow, ks);
    if (rc != TSN_OK) return rc;
    return copy_stats(ks, stats, cap, n_stats);
}

int tsn_synth_normal_f32(uint64_t seed, uint64_t index, double mean, double std, size_t n, float *out) {
    if (!out && n) { tsn::set_error("null output"); return TSN_ERR_ARG; }
    tsn::synth_normal_f32(seed, index, mean, std, n, out);
    return TSN_OK;
}
int tsn_synth_normal_bf16(uint64_t seed, uint64_t index, double mean, double std, size_t n, uint16_t *out) {
    if (!out && n) { tsn::set_error("null output"); return TSN_ERR_ARG; }
    tsn::synth_normal_bf16(seed, index, mean, std, n, out);
    return TSN_OK;
}
int tsn_synth_uniform_f32(uint64_t seed, uint64_t index, double lo, double hi, size_t n, float *out) {
    if (!out && n) { tsn::set_error("null output"); return TSN_ERR_ARG; }
    tsn::synth_uniform_f32(seed, index, lo, hi, n, out);
    return TSN_OK;
}
int tsn_refdit_synth_weights(const tsn_refdit_spec *spec, uint64_t seed, double norm_mean, uint16_t *out) {
    if (!spec || !out) { tsn::set_error("null spec or output"); return TSN_ERR_ARG; }
    const auto m = tsn::refdit_manifest(to_ref_spec(spec));
    for (size_t i = 0; i < m.size(); ++i) {
        const bool is_norm = m[i].name.find("norm.weight") != std::string::npos;
        tsn::synth_normal_bf16(seed, (uint64_t)i, is_norm ? norm_mean : 0.0, 0.02, (size_t)m[i].numel, out + m[i].offset);
    }
    return TSN_OK;
}
int tsn_refcond_synth_weights(const tsn_refcond_spec *spec, uint64_t seed, uint16_t *out) {
    if (!spec || !out) { tsn::set_error("null spec or output"); return TSN_ERR_ARG; }
    const auto m = tsn::refcond_manifest(to_cond_spec(spec));
    for (size_t i = 0; i < m.size(); ++i)
        tsn::synth_normal_bf16(seed, (uint64_t)i, 0.0, 0.02, (size_t)m[i].numel, out + m[i].offset);
    return TSN_OK;
}
int tsn_vae_synth_weights(const tsn_vae_spec *spec, uint64_t seed, float *out) {
    if (!spec || !out) { tsn::set_error("null spec or output"); return TSN_ERR_ARG; }
    const tsn::VaeSpec vs = to_vae_spec(spec);
    const auto m = tsn::vae_manifest(vs);
    for (size_t i = 0; i < m.size(); ++i) {
        const std::string &n = m[i].name;
        const bool snake = n.size() > 6 && (n.compare(n.size() - 6, 6, ".alpha") == 0 || n.compare(n.size() - 5, 5, ".beta") == 0);
        const bool bias = n.size() > 5 && n.compare(n.size() - 5, 5, ".bias") == 0;
        double std = 0.02;
        if (snake) std = 0.1;
        else if (!bias) {   // conv weight [OC][IC][K]: fan-in IC*K = numel / OC
            const int layer = atoi(n.c_str() + strlen("decoder.layers."));
            const int oc = layer == 0 ? vs.width[0] : layer == 7 ? vs.out_ch : vs.width[layer];
            std = 1.0 / sqrt((double)m[i].numel / oc);
            // the residual branch's closing k1 conv at half gain keeps the stream's scale bounded
            // over the 15 residual units (audio RMS near 1 instead of growing 2x per unit)
            if (n.size() > 16 && n.compare(n.size() - 16, 16, ".layers.3.weight") == 0) std *= 0.5;
        }
        tsn::synth_normal_f32(seed, (uint64_t)i, 0.0, std, (size_t)m[i].numel, out + m[i].offset);
    }
    return TSN_OK;
}
// per-tensor std of the encoders' synthetic weights (include/tsn.h): embeddings 1, norm weights 1 + 0.1,
// biases 0.02, residual-stream projections 0.5/sqrt(fan_in), other linears 1/sqrt(fan_in), rel bias 0.5
static void enc_synth(const std::vector<tsn::ManifestEntry> &m, uint64_t seed, float *out,
                      const std::function<int(const std::string &)> &fan_in) {
    for (size_t i = 0; i < m.size(); ++i) {
        const std::string &n = m[i].name;
        auto ends = [&](const char *suf) {
            const size_t k = strlen(suf);
            return n.size() >= k && n.compare(n.size() - k, k, suf) == 0;
        };
        double mean = 0.0, std = 0.02;
        if (n == "tok_emb" || n == "pos_emb") std = 1.0;
        else if (n == "rel_bias") std = 0.5;
        else if (ends("norm") || ends("ln1.w") || ends("ln2.w") || ends("out_ln.w")) { mean = 1.0; std = 0.1; }
        else if (ends(".b")) std = 0.02;
        else {
            const bool into_stream = ends(".out.w") || ends(".fc2.w") || ends(".o") || ends(".wo");
            std = (into_stream ? 0.5 : 1.0) / sqrt((double)fan_in(n));
        }
        tsn::synth_normal_f32(seed, (uint64_t)i, mean, std, (size_t)m[i].numel, out + m[i].offset);
    }
}
int tsn_clip_synth_weights(const tsn_clip_spec *spec, uint64_t seed, float *out) {
    if (!spec || !out) { tsn::set_error("null spec or output"); return TSN_ERR_ARG; }
    const tsn::ClipSpec s = to_clip_spec(spec);
    enc_synth(tsn::clip_manifest(s), seed, out, [&](const std::string &n) {
        const size_t k = n.size();
        return k >= 6 && n.compare(k - 6, 6, ".fc2.w") == 0 ? 4 * s.H : s.H;
    });
    return TSN_OK;
}
int tsn_t5_synth_weights(const tsn_t5_spec *spec, uint64_t seed, float *out) {
    if (!spec || !out) { tsn::set_error("null spec or output"); return TSN_ERR_ARG; }
    const tsn::T5Spec s = to_t5_spec(spec);
    enc_synth(tsn::t5_manifest(s), seed, out, [&](const std::string &n) {
        const size_t k = n.size();
        return k >= 3 && n.compare(k - 3, 3, ".wo") == 0 ? s.d_ff : s.d;
    });
    return TSN_OK;
}
int tsn_dit_synth_weights(const tsn_dit_spec *spec, uint64_t seed, double norm_mean, uint16_t *out) {
    if (!spec || !out) { tsn::set_error("null spec or output"); return TSN_ERR_ARG; }
    const auto m = tsn::dit_manifest(to_spec(spec));
    for (size_t i = 0; i < m.size(); ++i) {
        const bool is_norm = m[i].name.find("norm.weight") != std::string::npos;
        tsn::synth_normal_bf16(seed, (uint64_t)i, is_norm ? norm_mean : 0.0, 0.02, (size_t)m[i].numel, out + m[i].offset);
    }
    return TSN_OK;
}

} // extern "C"
