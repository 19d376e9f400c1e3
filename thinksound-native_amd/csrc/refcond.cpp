// refcond.cpp — RefCondModel: the reference's conditioning prep on HIP (src/dit.cpp:55-191).
#include "refcond.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <map>

#include "gguf.h"

namespace tsn {

std::vector<ManifestEntry> refcond_manifest(const RefCondSpec &s) {
    std::vector<ManifestEntry> v;
    const int64_t H = s.H, F = s.F;
    int64_t off = 0;
    auto add = [&](const std::string &n, int64_t numel) {
        v.push_back({n, numel, off});
        off += numel;
    };
    // SwiGLU MLP of taps-wide convs (taps 1: linear layers)
    auto swiglu = [&](const std::string &p, int64_t taps) {
        add(p + ".w1.weight", F * H * taps);
        add(p + ".w3.weight", F * H * taps);
        add(p + ".w2.weight", H * F * taps);
    };
    add("sync_pos_emb", 8 * (int64_t)s.sync_dim);
    add("sync_input_proj.0.weight", H * s.sync_dim * 7);
    add("sync_input_proj.0.bias", H);
    swiglu("sync_input_proj.2", 3);
    add("clip_input_proj.0.weight", H * s.clip_dim);
    add("clip_input_proj.0.bias", H);
    swiglu("clip_input_proj.2", 3);
    add("clip_cond_proj.weight", H * H);
    add("clip_cond_proj.bias", H);
    add("text_input_proj.0.weight", H * s.text_dim);
    add("text_input_proj.0.bias", H);
    swiglu("text_input_proj.2", 1);
    add("text_cond_proj.weight", H * s.gtext_dim);
    add("text_cond_proj.bias", H);
    swiglu("global_cond_mlp", 1);
    return v;
}

int refcond_spec_check(const RefCondSpec &s) {
    TSN_REQUIRE(s.T > 0 && s.C > 0 && s.sync_S > 0 && s.TS > 0, "refcond spec: T, C, sync_S, TS must be positive");
    TSN_REQUIRE(s.H % 256 == 0 && s.H > 0 && s.H <= 2048, "refcond spec: H must be a multiple of 256, <= 2048");
    TSN_REQUIRE(s.F % 64 == 0 && s.F > 0, "refcond spec: F must be a multiple of 64");
    TSN_REQUIRE(s.sync_dim % 64 == 0 && s.clip_dim % 64 == 0 && s.text_dim % 64 == 0 && s.sync_dim > 0 &&
                    s.clip_dim > 0 && s.text_dim > 0,
                "refcond spec: sync, clip and text widths must be multiples of 64");
    TSN_REQUIRE(s.gtext_dim % 8 == 0 && s.gtext_dim > 0, "refcond spec: pooled text width must be a multiple of 8");
    return TSN_OK;
}

RefCondSpec refcond_spec_for_duration(int dur_s) {
    RefCondSpec s{};
    s.H = 1024; s.F = 2816;
    s.T = (int)llround(44100.0 / 2048.0 * dur_s);
    s.C = 8 * dur_s;
    s.sync_S = 24 * dur_s;
    s.TS = 154;
    s.sync_dim = 768; s.clip_dim = 1024; s.text_dim = 2048; s.gtext_dim = 1024;
    return s;
}

int refcond_spec_from_gguf(const char *path, int T, int C, int sync_S, int TS, RefCondSpec *out) {
    TSN_REQUIRE(out, "refcond gguf: null spec");
    GgufReader g;
    TSN_TRY(g.open(path));
    RefCondSpec s = refcond_spec_for_duration(1);
    s.T = T; s.C = C; s.sync_S = sync_S; s.TS = TS;
    s.H = (int)g.get_i64("dit.hidden_dim", 1024);
    // widths from the input projections' shapes (ne[0] fastest): conv [OC][IC][K] -> (K, IC, OC)
    if (const GgufTensorInfo *t = g.find("sync_input_proj.2.w1.weight"))
        if (t->n_dims >= 3) s.F = (int)t->ne[2];
    if (const GgufTensorInfo *t = g.find("sync_input_proj.0.weight"))
        if (t->n_dims >= 3) s.sync_dim = (int)t->ne[1];
    if (const GgufTensorInfo *t = g.find("clip_input_proj.0.weight")) s.clip_dim = (int)t->ne[0];
    if (const GgufTensorInfo *t = g.find("text_input_proj.0.weight")) s.text_dim = (int)t->ne[0];
    if (const GgufTensorInfo *t = g.find("text_cond_proj.weight")) s.gtext_dim = (int)t->ne[0];
    TSN_TRY(refcond_spec_check(s));
    *out = s;
    return TSN_OK;
}

int RefCondModel::create(Runtime *r, const RefCondSpec &sp) {
    TSN_REQUIRE(r, "refcond: null runtime");
    TSN_TRY(refcond_spec_check(sp));
    rt = r;
    s = sp;
    const size_t H = s.H, F = s.F;
    const size_t rows = (size_t)std::max({s.sync_S, s.C, s.TS});
    const size_t in = std::max({(size_t)s.sync_S * s.sync_dim, (size_t)s.C * s.clip_dim, (size_t)s.TS * s.text_dim});
    TSN_TRY(alloc(in * 2 * sizeof(half_t), (void **)&IN_));
    TSN_TRY(alloc(rows * 2 * H * sizeof(half_t), (void **)&XA_));
    TSN_TRY(alloc(rows * 2 * F * sizeof(half_t), (void **)&HF_));
    TSN_TRY(alloc((size_t)s.sync_S * H * sizeof(float), (void **)&SMID_));
    TSN_TRY(alloc(H * sizeof(float), (void **)&cmean_));
    TSN_TRY(alloc(H * sizeof(float), (void **)&fc_));
    TSN_TRY(alloc(F * sizeof(float), (void **)&ga_));
    TSN_TRY(alloc(F * sizeof(float), (void **)&gb_));
    ws_bytes_ = (size_t)40 << 20;
    TSN_TRY(alloc(ws_bytes_, (void **)&ws_));
    TSN_TRY(alloc_skcnt());
    // latent row i takes sync row floor((i + 0.5) * sync_S / T), computed in f32 as src/dit.cpp:112
    std::vector<int32_t> idx(s.T);
    for (int i = 0; i < s.T; ++i) {
        const int si = (int)floorf(((float)i + 0.5f) * (float)s.sync_S / (float)s.T);
        idx[i] = std::min(std::max(si, 0), s.sync_S - 1);
    }
    TSN_TRY(alloc(idx.size() * sizeof(int32_t), (void **)&idx_));
    TSN_TRY(rt->dev.upload(idx_, idx.data(), idx.size() * sizeof(int32_t)));
    return TSN_OK;
}

int RefCondModel::upload_weights(const uint16_t *host, size_t numel) { return upload(host, false, numel); }
int RefCondModel::upload_weights_f32(const float *host, size_t numel) { return upload(host, true, numel); }

int RefCondModel::load_gguf(const char *path) {
    GgufReader g;
    TSN_TRY(g.open(path));
    std::vector<float> host;
    TSN_TRY(gguf_read_manifest(g, refcond_manifest(s), host));
    return upload(host.data(), true, host.size());
}

int RefCondModel::upload(const void *host, bool src_f32, size_t numel) {
    TSN_REQUIRE(rt && host, "refcond: not created / null weights");
    TSN_REQUIRE(!ready_, "refcond: weights already uploaded");
    const auto man = refcond_manifest(s);
    const size_t total = (size_t)(man.back().offset + man.back().numel);
    TSN_REQUIRE(numel == total, "refcond: weight count does not match the manifest (" + std::to_string(total) + ")");
    const size_t esz = src_f32 ? 4 : 2;
    TSN_TRY(alloc(total * esz, &wraw_));
    TSN_TRY(rt->dev.upload(wraw_, host, total * esz));
    std::map<std::string, const ManifestEntry *> idx;
    for (const auto &e : man) idx[e.name] = &e;
    const hipStream_t st = rt->dev.stream();
    const int H = s.H, F = s.F;
    auto prep = [&](const std::string &n, int OC, int IC, int KT, int ra, int rb, int rc, int rd, void *dst,
                    long long dst_rows, int out_f32) -> int {
        TSN_REQUIRE(idx.at(n)->numel == (int64_t)OC * IC * KT, "refcond: tensor size mismatch: " + n);
        return launch_weight_prep((const char *)wraw_ + idx.at(n)->offset * esz, src_f32 ? 1 : 0, dst, out_f32, OC,
                                  IC, KT, 0, ra, rb, rc, rd, dst_rows, st);
    };
    auto f16w = [&](const std::string &n, int OC, int IC, int KT, const half_t **out) -> int {
        half_t *p;
        TSN_TRY(alloc((size_t)OC * IC * KT * 2, (void **)&p));
        TSN_TRY(prep(n, OC, IC, KT, 1, 0, 1, 0, p, OC, 0));
        *out = p;
        return TSN_OK;
    };
    auto f32v = [&](const std::string &n, int N, const float **out) -> int {
        float *p;
        TSN_TRY(alloc((size_t)N * 4, (void **)&p));
        TSN_TRY(prep(n, N, 1, 1, 1, 0, 1, 0, p, N, 1));
        *out = p;
        return TSN_OK;
    };
    // w1, w3 [F][IC][KT] -> [2F][KT][IC] in 64-row blocks (w1 block j, w3 block j) for the SwiGLU epilogue
    auto swiglu_w = [&](const std::string &p, int KT, const half_t **w13, const half_t **w2) -> int {
        half_t *w;
        TSN_TRY(alloc((size_t)2 * F * H * KT * 2, (void **)&w));
        TSN_TRY(prep(p + ".w1.weight", F, H, KT, 64, 1, 128, 0, w, 2LL * F, 0));
        TSN_TRY(prep(p + ".w3.weight", F, H, KT, 64, 1, 128, 64, w, 2LL * F, 0));
        *w13 = w;
        return f16w(p + ".w2.weight", H, F, KT, w2);
    };
    TSN_TRY(f32v("sync_pos_emb", 8 * s.sync_dim, &pe_));
    TSN_TRY(f16w("sync_input_proj.0.weight", H, s.sync_dim, 7, &Ws0_));
    TSN_TRY(f32v("sync_input_proj.0.bias", H, &bs0_));
    TSN_TRY(swiglu_w("sync_input_proj.2", 3, &W13s_, &W2s_));
    TSN_TRY(f16w("clip_input_proj.0.weight", H, s.clip_dim, 1, &Wc0_));
    TSN_TRY(f32v("clip_input_proj.0.bias", H, &bc0_));
    TSN_TRY(swiglu_w("clip_input_proj.2", 3, &W13c_, &W2c_));
    TSN_TRY(f16w("clip_cond_proj.weight", H, H, 1, &Wcfc_));
    TSN_TRY(f32v("clip_cond_proj.bias", H, &bcfc_));
    TSN_TRY(f16w("text_input_proj.0.weight", H, s.text_dim, 1, &Wt0_));
    TSN_TRY(f32v("text_input_proj.0.bias", H, &bt0_));
    TSN_TRY(swiglu_w("text_input_proj.2", 1, &W13t_, &W2t_));
    TSN_TRY(f16w("text_cond_proj.weight", H, s.gtext_dim, 1, &Wtfc_));
    TSN_TRY(f32v("text_cond_proj.bias", H, &btfc_));
    TSN_TRY(f16w("global_cond_mlp.w1.weight", F, H, 1, &Wg1_));
    TSN_TRY(f16w("global_cond_mlp.w3.weight", F, H, 1, &Wg3_));
    TSN_TRY(f16w("global_cond_mlp.w2.weight", H, F, 1, &Wg2_));
    TSN_TRY(rt->dev.sync());
    TSN_TRY(release(wraw_));
    wraw_ = nullptr;
    ready_ = true;
    return TSN_OK;
}

namespace {
void half_w(GemmProblem &p) {
    p.w_half = 1;
    p.ldw = p.taps * p.Kc / 2;
}
} // namespace

// IN [rows][2K] hi|lo -> conv (taps, pad taps/2) or linear + b -> SiLU -> XA [rows][2H] hi|lo
int RefCondModel::proj_silu(int rows, int K, int taps, const half_t *W, const float *b) {
    GemmBatch g;
    g.nprob = 1;
    store_problem(g.p[0], IN_, 2 * K, RowMap{rows, rows, 0}, taps, 2 * K, rows, s.H, W, XA_, 2 * s.H, 1);
    g.p[0].bias = b;
    g.p[0].y_lo = s.H;
    half_w(g.p[0]);
    g.ws = ws_;
    g.ws_bytes = ws_bytes_;
    return gemm_run(g, EPI_STORE);
}

// XA [rows][2H] hi|lo -> SwiGLU (w1|w3) -> HF [rows][2F] hi|lo -> w2 -> y [rows][H] f32
int RefCondModel::swiglu_mlp(int rows, int taps, const half_t *W13, const half_t *W2, float *y) {
    const RowMap D{rows, rows, 0};
    GemmBatch a;
    a.nprob = 1;
    store_problem(a.p[0], XA_, 2 * s.H, D, taps, 2 * s.H, rows, 2 * s.F, W13, HF_, 2 * s.F, 0);
    a.p[0].y_lo = s.F;
    half_w(a.p[0]);
    a.ws = ws_;
    a.ws_bytes = ws_bytes_;
    TSN_TRY(gemm_run(a, EPI_SWIGLU));
    GemmBatch b;
    b.nprob = 1;
    store_problem(b.p[0], HF_, 2 * s.F, D, taps, 2 * s.F, rows, s.H, W2, nullptr, 0, 0);
    b.p[0].Y = y; b.p[0].ldy = s.H; b.p[0].y_f16 = 0;
    half_w(b.p[0]);
    b.ws = ws_;
    b.ws_bytes = ws_bytes_;
    return gemm_run(b, EPI_STORE);
}

// src/dit.cpp:91-134
int RefCondModel::enqueue_prep_conditioning(const float *clip_f, const float *sync_f, float *clip_pp,
                                            float *sync_gather, float *clip_fc) {
    TSN_REQUIRE(ready_, "refcond: weights not uploaded");
    TSN_REQUIRE(clip_f && sync_f && clip_pp && sync_gather && clip_fc, "refcond prep: null argument");
    TSN_TRY(rt->dev.make_current());
    const hipStream_t st = rt->dev.stream();
    const int H = s.H;
    // sync: + positional embedding (period 8) -> conv k7 pad 3 + b -> SiLU -> SwiGLU conv-MLP -> gather
    TSN_TRY(run("add_period_hilo_kernel", 0, 8.0 * s.sync_S * s.sync_dim, [&] {
        return launch_add_period_hilo(sync_f, pe_, 8, IN_, s.sync_S, s.sync_dim, st);
    }));
    TSN_TRY(proj_silu(s.sync_S, s.sync_dim, 7, Ws0_, bs0_));
    TSN_TRY(swiglu_mlp(s.sync_S, 3, W13s_, W2s_, SMID_));
    TSN_TRY(run("gather_rows_kernel", 0, 8.0 * s.T * H, [&] { return launch_gather_rows(SMID_, idx_, sync_gather, s.T, H, st); }));
    // clip: linear + b -> SiLU -> SwiGLU conv-MLP; clip_fc from the row mean
    TSN_TRY(run("add_period_hilo_kernel", 0, 8.0 * s.C * s.clip_dim, [&] {
        return launch_add_period_hilo(clip_f, nullptr, 1, IN_, s.C, s.clip_dim, st);
    }));
    TSN_TRY(proj_silu(s.C, s.clip_dim, 1, Wc0_, bc0_));
    TSN_TRY(swiglu_mlp(s.C, 3, W13c_, W2c_, clip_pp));
    TSN_TRY(run("mean_rows_kernel", 0, 4.0 * s.C * H, [&] { return launch_mean_rows(clip_pp, s.C, H, cmean_, st); }));
    GemvArgs g;
    memset(&g, 0, sizeof g);
    g.W = Wcfc_; g.ldw = H; g.wdt = DT_F16; g.X = cmean_; g.ldx = H; g.Y = clip_fc; g.ldy = H;
    g.bias = bcfc_; g.N = H; g.K = H; g.nb = 1;
    return run(K_GEMV, 2.0 * H * H, 2.0 * H * H, [&] { return launch_gemv(g, st); });
}

// src/dit.cpp:137-191
int RefCondModel::enqueue_prep_text_arm(const float *text_cat, const float *gtext, const float *clip_fc,
                                        float *text_pp, float *gcmlp) {
    TSN_REQUIRE(ready_, "refcond: weights not uploaded");
    TSN_REQUIRE(text_cat && gtext && clip_fc && text_pp && gcmlp, "refcond text arm: null argument");
    TSN_TRY(rt->dev.make_current());
    const hipStream_t st = rt->dev.stream();
    const int H = s.H, F = s.F;
    TSN_TRY(run("add_period_hilo_kernel", 0, 8.0 * s.TS * s.text_dim, [&] {
        return launch_add_period_hilo(text_cat, nullptr, 1, IN_, s.TS, s.text_dim, st);
    }));
    TSN_TRY(proj_silu(s.TS, s.text_dim, 1, Wt0_, bt0_));
    TSN_TRY(swiglu_mlp(s.TS, 1, W13t_, W2t_, text_pp));
    // fc = text_cond_proj(gtext) + b + clip_fc; gcmlp = w2(silu(w1 fc) * (w3 fc)), all f32
    auto gemv = [&](const half_t *W, int N, int K, const float *x, float *y, const float *bias, const float *addv) {
        GemvArgs g;
        memset(&g, 0, sizeof g);
        g.W = W; g.ldw = K; g.wdt = DT_F16; g.X = x; g.ldx = K; g.Y = y; g.ldy = N;
        g.bias = bias; g.addv = addv; g.ld_add = N; g.N = N; g.K = K; g.nb = 1;
        return run(K_GEMV, 2.0 * N * K, 2.0 * N * K, [&] { return launch_gemv(g, st); });
    };
    TSN_TRY(gemv(Wtfc_, H, s.gtext_dim, gtext, fc_, btfc_, clip_fc));
    TSN_TRY(gemv(Wg1_, F, H, fc_, ga_, nullptr, nullptr));
    TSN_TRY(gemv(Wg3_, F, H, fc_, gb_, nullptr, nullptr));
    TSN_TRY(run("swiglu_kernel", 0, 12.0 * F, [&] { return launch_swiglu(ga_, gb_, ga_, (size_t)F, st); }));
    return gemv(Wg2_, H, F, ga_, gcmlp, nullptr, nullptr);
}

} // namespace tsn
