// encoders.cpp — ClipModel and T5Model: the reference's text encoders on HIP (src/clip.cpp, src/t5.cpp).
#include "encoders.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <map>

#include "gguf.h"

namespace tsn {

namespace {

struct Layout {   // device arena: named regions at float offsets
    std::map<std::string, size_t> at;
    size_t size = 0;
    size_t put(const std::string &n, size_t numel) {
        at[n] = size;
        size += (numel + 3) & ~(size_t)3;   // 16-byte aligned regions
        return at[n];
    }
};

// stage the host tensors into the arena layout (the tensors of `group` go one after the other at
// the region of group[0]), upload once
int fill_arena(Runtime *rt, const std::vector<ManifestEntry> &man, const float *host, const Layout &lay,
               const std::map<std::string, std::pair<std::string, size_t>> &group, float *dev) {
    std::vector<float> stage(lay.size, 0.0f);
    for (const auto &e : man) {
        size_t dst;
        const auto g = group.find(e.name);
        if (g != group.end()) dst = lay.at.at(g->second.first) + g->second.second;
        else dst = lay.at.at(e.name);
        memcpy(stage.data() + dst, host + e.offset, (size_t)e.numel * sizeof(float));
    }
    return rt->dev.upload(dev, stage.data(), stage.size() * sizeof(float));
}

} // namespace

int t5_bucket(int rel, int n_bucket, int max_dist) {
    const int half = n_bucket / 2;
    int b = rel > 0 ? half : 0;
    const int n = rel < 0 ? -rel : rel;
    const int exact = half / 2;
    if (n < exact) return b + n;
    const int v = exact + (int)(log((double)n / exact) / log((double)max_dist / exact) * (half - exact));
    return b + std::min(v, half - 1);
}

/* ---------------- specs and manifests ---------------- */

ClipSpec clip_spec_default() { return ClipSpec{1024, 24, 16, 77, 49408, 1e-5f}; }
T5Spec t5_spec_default() { return T5Spec{2048, 5120, 24, 32, 77, 32128, 32, 128, 1e-6f}; }

int clip_spec_check(const ClipSpec &s) {
    TSN_REQUIRE(s.H > 0 && s.H % 64 == 0 && s.NH * 64 == s.H, "clip spec: heads of 64 (H = 64 NH)");
    TSN_REQUIRE(s.NL > 0 && s.ctx > 0 && s.ctx <= 128 && s.vocab > 0, "clip spec: layers, context 1..128, vocabulary");
    return TSN_OK;
}

int t5_spec_check(const T5Spec &s) {
    TSN_REQUIRE(s.d > 0 && s.d % 64 == 0 && s.NH * 64 == s.d, "t5 spec: heads of 64 (d = 64 NH)");
    TSN_REQUIRE(s.d_ff > 0 && s.d_ff % 32 == 0, "t5 spec: d_ff a multiple of 32");
    TSN_REQUIRE(s.NL > 0 && s.ctx > 0 && s.ctx <= 128 && s.vocab > 0, "t5 spec: layers, context 1..128, vocabulary");
    TSN_REQUIRE(s.n_bucket >= 4 && s.n_bucket % 4 == 0 && s.max_dist > s.n_bucket / 4,
                "t5 spec: relative buckets (a multiple of 4) and a max distance past the exact range");
    return TSN_OK;
}

int clip_spec_from_gguf(const char *path, ClipSpec *out) {
    TSN_REQUIRE(out, "clip gguf: null spec");
    GgufReader g;
    TSN_TRY(g.open(path));
    ClipSpec s = clip_spec_default();
    s.H = (int)g.get_i64("clip.hidden", s.H);
    s.NL = (int)g.get_i64("clip.layers", s.NL);
    s.NH = (int)g.get_i64("clip.heads", s.NH);
    s.ctx = (int)g.get_i64("clip.ctx", s.ctx);
    if (const GgufTensorInfo *t = g.find("tok_emb")) s.vocab = (int)t->ne[1];
    TSN_TRY(clip_spec_check(s));
    *out = s;
    return TSN_OK;
}

int t5_spec_from_gguf(const char *path, T5Spec *out) {
    TSN_REQUIRE(out, "t5 gguf: null spec");
    GgufReader g;
    TSN_TRY(g.open(path));
    T5Spec s = t5_spec_default();
    s.d = (int)g.get_i64("t5.d_model", s.d);
    s.d_ff = (int)g.get_i64("t5.d_ff", s.d_ff);
    s.NL = (int)g.get_i64("t5.n_layers", s.NL);
    s.NH = (int)g.get_i64("t5.n_heads", s.NH);
    s.n_bucket = (int)g.get_i64("t5.rel_buckets", s.n_bucket);
    s.max_dist = (int)g.get_i64("t5.rel_max_dist", s.max_dist);
    s.eps = (float)g.get_f64("t5.eps", s.eps);
    if (const GgufTensorInfo *t = g.find("tok_emb")) s.vocab = (int)t->ne[1];
    TSN_TRY(t5_spec_check(s));
    *out = s;
    return TSN_OK;
}

std::vector<ManifestEntry> clip_manifest(const ClipSpec &s) {
    std::vector<ManifestEntry> v;
    int64_t off = 0;
    auto add = [&](const std::string &n, int64_t numel) {
        v.push_back({n, numel, off});
        off += numel;
    };
    const int64_t H = s.H;
    add("tok_emb", (int64_t)s.vocab * H);
    add("pos_emb", (int64_t)s.ctx * H);
    for (int l = 0; l < s.NL; ++l) {
        const std::string b = "blk." + std::to_string(l);
        add(b + ".ln1.w", H); add(b + ".ln1.b", H);
        add(b + ".q.w", H * H); add(b + ".q.b", H);
        add(b + ".k.w", H * H); add(b + ".k.b", H);
        add(b + ".v.w", H * H); add(b + ".v.b", H);
        add(b + ".out.w", H * H); add(b + ".out.b", H);
        add(b + ".ln2.w", H); add(b + ".ln2.b", H);
        add(b + ".fc1.w", 4 * H * H); add(b + ".fc1.b", 4 * H);
        add(b + ".fc2.w", H * 4 * H); add(b + ".fc2.b", H);
    }
    add("out_ln.w", H);
    add("out_ln.b", H);
    add("text_proj", H * H);
    return v;
}

std::vector<ManifestEntry> t5_manifest(const T5Spec &s) {
    std::vector<ManifestEntry> v;
    int64_t off = 0;
    auto add = [&](const std::string &n, int64_t numel) {
        v.push_back({n, numel, off});
        off += numel;
    };
    const int64_t d = s.d, F = s.d_ff;
    add("tok_emb", (int64_t)s.vocab * d);
    for (int l = 0; l < s.NL; ++l) {
        const std::string b = "blk." + std::to_string(l);
        add(b + ".attn_norm", d);
        add(b + ".q", d * d); add(b + ".k", d * d); add(b + ".v", d * d); add(b + ".o", d * d);
        add(b + ".ffn_norm", d);
        add(b + ".wi_0", F * d); add(b + ".wi_1", F * d); add(b + ".wo", d * F);
    }
    add("rel_bias", (int64_t)s.n_bucket * s.NH);
    add("out_norm", d);
    return v;
}

/* ---------------- CLIP ---------------- */

int ClipModel::create(Runtime *r, const ClipSpec &sp) {
    TSN_REQUIRE(r, "clip: null runtime");
    TSN_TRY(clip_spec_check(sp));
    rt = r;
    s = sp;
    const size_t n = s.ctx, H = s.H;
    TSN_TRY(alloc(n * H * 4, (void **)&X_));
    TSN_TRY(alloc(n * H * 4, (void **)&R_));
    TSN_TRY(alloc(n * 3 * H * 4, (void **)&QKV_));
    TSN_TRY(alloc(n * H * 4, (void **)&ATT_));
    TSN_TRY(alloc(n * 4 * H * 4, (void **)&FF_));
    TSN_TRY(alloc(n * 4, (void **)&ids_));
    TSN_TRY(alloc(ENC_WS_BYTES, (void **)&ws_));
    return TSN_OK;
}

int ClipModel::upload_weights(const float *host, size_t numel) { return upload(host, numel); }

int ClipModel::load_gguf(const char *path) {
    GgufReader g;
    TSN_TRY(g.open(path));
    std::vector<float> host;
    TSN_TRY(gguf_read_manifest(g, clip_manifest(s), host));
    return upload(host.data(), host.size());
}

int ClipModel::upload(const float *host, size_t numel) {
    TSN_REQUIRE(rt && host, "clip: not created / null weights");
    TSN_REQUIRE(!ready_, "clip: weights already uploaded");
    const auto man = clip_manifest(s);
    const size_t total = (size_t)(man.back().offset + man.back().numel);
    TSN_REQUIRE(numel == total, "clip: weight count does not match the manifest (" + std::to_string(total) + ")");
    const size_t H = s.H;
    Layout lay;
    std::map<std::string, std::pair<std::string, size_t>> group;
    for (const auto &e : man) {
        const std::string &n = e.name;
        const std::string stem = n.compare(0, 4, "blk.") == 0 ? n.substr(0, n.find('.', 4)) : "";
        const std::string leaf = stem.empty() ? n : n.substr(stem.size() + 1);
        if (leaf == "q.w" || leaf == "k.w" || leaf == "v.w") {   // one [3H][H] weight per layer
            const size_t j = leaf[0] == 'q' ? 0 : leaf[0] == 'k' ? 1 : 2;
            if (j == 0) lay.put(stem + ".qkv.w", 3 * H * H);
            group[n] = {stem + ".qkv.w", j * H * H};
        } else if (leaf == "q.b" || leaf == "k.b" || leaf == "v.b") {
            const size_t j = leaf[0] == 'q' ? 0 : leaf[0] == 'k' ? 1 : 2;
            if (j == 0) lay.put(stem + ".qkv.b", 3 * H);
            group[n] = {stem + ".qkv.b", j * H};
        } else {
            lay.put(n, (size_t)e.numel);
        }
    }
    float *dev;
    TSN_TRY(alloc(lay.size * sizeof(float), (void **)&dev));
    TSN_TRY(fill_arena(rt, man, host, lay, group, dev));
    auto P = [&](const std::string &n) { return (const float *)(dev + lay.at.at(n)); };
    tok_ = P("tok_emb");
    pos_ = P("pos_emb");
    L_.resize(s.NL);
    for (int l = 0; l < s.NL; ++l) {
        const std::string b = "blk." + std::to_string(l);
        L_[l] = Layer{P(b + ".ln1.w"), P(b + ".ln1.b"), P(b + ".qkv.w"), P(b + ".qkv.b"), P(b + ".out.w"),
                      P(b + ".out.b"), P(b + ".ln2.w"), P(b + ".ln2.b"), P(b + ".fc1.w"), P(b + ".fc1.b"),
                      P(b + ".fc2.w"), P(b + ".fc2.b")};
    }
    lnw_ = P("out_ln.w");
    lnb_ = P("out_ln.b");
    proj_ = P("text_proj");
    ready_ = true;
    return TSN_OK;
}

int ClipModel::encode(const int32_t *ids, float *per_token, float *global) {
    TSN_REQUIRE(ready_, "clip: weights not uploaded");
    TSN_REQUIRE(ids && per_token && global, "clip: null ids or outputs");
    const int n = s.ctx, H = s.H;
    int eos = 0;
    for (int i = 0; i < n; ++i) {
        TSN_REQUIRE(ids[i] >= 0 && ids[i] < s.vocab, "clip: token id outside the vocabulary");
        if (ids[i] > ids[eos]) eos = i;   // first position of the largest id (src/clip.cpp:45-46)
    }
    TSN_TRY(rt->dev.upload(ids_, ids, (size_t)n * 4));
    const hipStream_t st = rt->dev.stream();
    auto gemm = [&](const float *A, int lda, const float *W, const float *b, float *Y, int ldy, int M, int N, int K,
                    int resid, int act) {
        EncGemmArgs g{A, lda, W, K, b, Y, ldy, M, N, K, resid, act, ws_, ENC_WS_BYTES, 1, 0};
        return run("gemm_f32_kernel", 2.0 * M * N * K, 4.0 * ((double)N * K + (double)M * K + M * (double)N),
                   [&] { return launch_gemm_f32(g, st); });
    };
    auto norm = [&](const float *x, float *y, const float *w, const float *b) {
        return run("enc_norm_kernel<true>", 0, 8.0 * n * H, [&] { return launch_enc_norm(x, y, w, b, n, H, s.eps, true, st); });
    };
    TSN_TRY(run("embed_rows_kernel", 0, 12.0 * n * H, [&] { return launch_embed_rows(ids_, tok_, pos_, X_, n, H, st); }));
    for (int l = 0; l < s.NL; ++l) {
        const Layer &w = L_[l];
        TSN_TRY(norm(X_, R_, w.ln1w, w.ln1b));
        TSN_TRY(gemm(R_, H, w.Wqkv, w.bqkv, QKV_, 3 * H, n, 3 * H, H, 0, 0));
        EncAttnArgs a{QKV_, 3 * H, 0, H, 2 * H, ATT_, H, n, s.NH, 64, 0.125f, 2, nullptr, nullptr, nullptr, eos};
        TSN_TRY(run("enc_attn_kernel", 4.0 * s.NH * n * (double)n * 64, 16.0 * n * H,
                    [&] { return launch_enc_attention(a, st); }));
        TSN_TRY(gemm(ATT_, H, w.Wo, w.bo, X_, H, n, H, H, 1, 0));
        TSN_TRY(norm(X_, R_, w.ln2w, w.ln2b));
        TSN_TRY(gemm(R_, H, w.W1, w.b1, FF_, 4 * H, n, 4 * H, H, 0, 1));
        TSN_TRY(gemm(FF_, 4 * H, w.W2, w.b2, X_, H, n, H, 4 * H, 1, 0));
    }
    TSN_TRY(norm(X_, per_token, lnw_, lnb_));
    // pooled: text_proj · per_token[eos] (src/clip.cpp:88-91)
    return gemm(per_token + (size_t)eos * H, H, proj_, nullptr, global, H, 1, H, H, 0, 0);
}

/* ---------------- T5 ---------------- */

int T5Model::create(Runtime *r, const T5Spec &sp) {
    TSN_REQUIRE(r, "t5: null runtime");
    TSN_TRY(t5_spec_check(sp));
    rt = r;
    s = sp;
    const size_t n = s.ctx, d = s.d, F = s.d_ff;
    TSN_TRY(alloc(n * d * 4, (void **)&X_));
    TSN_TRY(alloc(n * d * 4, (void **)&R_));
    TSN_TRY(alloc(n * 3 * d * 4, (void **)&QKV_));
    TSN_TRY(alloc(n * d * 4, (void **)&ATT_));
    TSN_TRY(alloc(n * 2 * F * 4, (void **)&U_));
    TSN_TRY(alloc(n * F * 4, (void **)&G_));
    TSN_TRY(alloc(n * 4, (void **)&ids_));
    TSN_TRY(alloc(n * 4, (void **)&pad_));
    TSN_TRY(alloc(ENC_WS_BYTES, (void **)&ws_));
    // bucket of (q, k) = bucket(k - q) (src/t5.cpp:47-53)
    std::vector<int32_t> bk(n * n);
    for (size_t q = 0; q < n; ++q)
        for (size_t k = 0; k < n; ++k) bk[q * n + k] = t5_bucket((int)k - (int)q, s.n_bucket, s.max_dist);
    TSN_TRY(alloc(bk.size() * 4, (void **)&bucket_));
    TSN_TRY(rt->dev.upload(bucket_, bk.data(), bk.size() * 4));
    return TSN_OK;
}

int T5Model::upload_weights(const float *host, size_t numel) { return upload(host, numel); }

int T5Model::load_gguf(const char *path) {
    GgufReader g;
    TSN_TRY(g.open(path));
    std::vector<float> host;
    TSN_TRY(gguf_read_manifest(g, t5_manifest(s), host));
    return upload(host.data(), host.size());
}

int T5Model::upload(const float *host, size_t numel) {
    TSN_REQUIRE(rt && host, "t5: not created / null weights");
    TSN_REQUIRE(!ready_, "t5: weights already uploaded");
    const auto man = t5_manifest(s);
    const size_t total = (size_t)(man.back().offset + man.back().numel);
    TSN_REQUIRE(numel == total, "t5: weight count does not match the manifest (" + std::to_string(total) + ")");
    const size_t d = s.d, F = s.d_ff;
    Layout lay;
    std::map<std::string, std::pair<std::string, size_t>> group;
    for (const auto &e : man) {
        const std::string &n = e.name;
        const std::string stem = n.compare(0, 4, "blk.") == 0 ? n.substr(0, n.find('.', 4)) : "";
        const std::string leaf = stem.empty() ? n : n.substr(stem.size() + 1);
        if (leaf == "q" || leaf == "k" || leaf == "v") {
            const size_t j = leaf == "q" ? 0 : leaf == "k" ? 1 : 2;
            if (j == 0) lay.put(stem + ".qkv", 3 * d * d);
            group[n] = {stem + ".qkv", j * d * d};
        } else if (leaf == "wi_0" || leaf == "wi_1") {   // one [2F][d] weight: wi_0 rows, then wi_1 rows
            const size_t j = leaf == "wi_0" ? 0 : 1;
            if (j == 0) lay.put(stem + ".wi", 2 * F * d);
            group[n] = {stem + ".wi", j * F * d};
        } else {
            lay.put(n, (size_t)e.numel);
        }
    }
    float *dev;
    TSN_TRY(alloc(lay.size * sizeof(float), (void **)&dev));
    TSN_TRY(fill_arena(rt, man, host, lay, group, dev));
    auto P = [&](const std::string &n) { return (const float *)(dev + lay.at.at(n)); };
    tok_ = P("tok_emb");
    L_.resize(s.NL);
    for (int l = 0; l < s.NL; ++l) {
        const std::string b = "blk." + std::to_string(l);
        L_[l] = Layer{P(b + ".attn_norm"), P(b + ".qkv"), P(b + ".o"), P(b + ".ffn_norm"), P(b + ".wi"), P(b + ".wo")};
    }
    rel_ = P("rel_bias");
    on_ = P("out_norm");
    ready_ = true;
    return TSN_OK;
}

int T5Model::encode(const int32_t *ids, float *out) {
    TSN_REQUIRE(ready_, "t5: weights not uploaded");
    TSN_REQUIRE(ids && out, "t5: null ids or output");
    const int n = s.ctx, d = s.d, F = s.d_ff;
    std::vector<int32_t> pad((size_t)n);
    for (int i = 0; i < n; ++i) {
        TSN_REQUIRE(ids[i] >= 0 && ids[i] < s.vocab, "t5: token id outside the vocabulary");
        pad[i] = ids[i] != 0;   // keys of id 0 (pad) masked (src/t5.cpp:90-94)
    }
    TSN_TRY(rt->dev.upload(ids_, ids, (size_t)n * 4));
    TSN_TRY(rt->dev.upload(pad_, pad.data(), (size_t)n * 4));
    const hipStream_t st = rt->dev.stream();
    auto gemm = [&](const float *A, int lda, const float *W, float *Y, int ldy, int M, int N, int K, int resid) {
        EncGemmArgs g{A, lda, W, K, nullptr, Y, ldy, M, N, K, resid, 0, ws_, ENC_WS_BYTES, 1, 0};
        return run("gemm_f32_kernel", 2.0 * M * N * K, 4.0 * ((double)N * K + (double)M * K + M * (double)N),
                   [&] { return launch_gemm_f32(g, st); });
    };
    auto rms = [&](const float *x, float *y, const float *w) {
        return run("enc_norm_kernel<false>", 0, 8.0 * n * d,
                   [&] { return launch_enc_norm(x, y, w, nullptr, n, d, s.eps, false, st); });
    };
    TSN_TRY(run("embed_rows_kernel", 0, 8.0 * n * d, [&] { return launch_embed_rows(ids_, tok_, nullptr, X_, n, d, st); }));
    for (int l = 0; l < s.NL; ++l) {
        const Layer &w = L_[l];
        TSN_TRY(rms(X_, R_, w.an));
        TSN_TRY(gemm(R_, d, w.Wqkv, QKV_, 3 * d, n, 3 * d, d, 0));
        // scale 1: T5 folds 1/sqrt(d_kv) into q (src/t5.cpp:70)
        EncAttnArgs a{QKV_, 3 * d, 0, d, 2 * d, ATT_, d, n, s.NH, 64, 1.0f, 1, bucket_, rel_, pad_, 0};
        TSN_TRY(run("enc_attn_kernel", 4.0 * s.NH * n * (double)n * 64, 16.0 * n * d,
                    [&] { return launch_enc_attention(a, st); }));
        TSN_TRY(gemm(ATT_, d, w.Wo, X_, d, n, d, d, 1));
        TSN_TRY(rms(X_, R_, w.fn));
        TSN_TRY(gemm(R_, d, w.Wi, U_, 2 * F, n, 2 * F, d, 0));
        TSN_TRY(run("geglu_rows_kernel", 0, 12.0 * n * F, [&] { return launch_geglu_rows(U_, G_, n, F, st); }));
        TSN_TRY(gemm(G_, F, w.Wout, X_, d, n, d, F, 1));
    }
    return rms(X_, out, on_);
}

} // namespace tsn
