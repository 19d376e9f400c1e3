// oracle_cond.cpp — CPU f32 restatement of the reference's conditioning prep (test infrastructure
// only): DitModel::prep_conditioning and DitModel::prep_text_arm (src/dit.cpp:55-192).
//
//   sync:  sync_f [sync_S, 768] + sync_pos_emb[s % 8] -> conv k7 pad 3 (768 -> H) + b -> SiLU ->
//          SwiGLU conv-MLP (k3) -> row i of sync_gather [T, H] is row floor((i + 0.5)*sync_S/T)
//          (src/dit.cpp:91-116);
//   clip:  clip_f [C, 1024] -> linear + b -> SiLU -> SwiGLU conv-MLP = clip_pp [C, H];
//          clip_fc = clip_cond_proj(mean over rows of clip_pp) (src/dit.cpp:118-134);
//   text arm: text_cat [TS, 2048] -> linear + b -> SiLU -> SwiGLU MLP (linear) = text_pp [TS, H];
//          gcmlp = SwiGLU MLP(text_cond_proj(gtext) + clip_fc), one row (src/dit.cpp:137-191).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "oracle.h"

namespace {

struct Tensor { std::string name; int64_t numel; };

// Weight manifest of the conditioning prep, in flat-buffer order. Conv weights [OC][IC][K],
// linear weights [N][K].
std::vector<Tensor> cond_manifest(const orc_refcond_spec &s) {
    std::vector<Tensor> v;
    const int64_t H = s.H, F = s.F;
    auto add = [&](const std::string &n, int64_t numel) { v.push_back({n, numel}); };
    auto convmlp = [&](const std::string &p) {
        add(p + ".w1.weight", F * H * 3);
        add(p + ".w3.weight", F * H * 3);
        add(p + ".w2.weight", H * F * 3);
    };
    auto mlp = [&](const std::string &p) {
        add(p + ".w1.weight", F * H);
        add(p + ".w3.weight", F * H);
        add(p + ".w2.weight", H * F);
    };
    add("sync_pos_emb", 8 * (int64_t)s.sync_dim);
    add("sync_input_proj.0.weight", H * s.sync_dim * 7);
    add("sync_input_proj.0.bias", H);
    convmlp("sync_input_proj.2");
    add("clip_input_proj.0.weight", H * s.clip_dim);
    add("clip_input_proj.0.bias", H);
    convmlp("clip_input_proj.2");
    add("clip_cond_proj.weight", H * H);
    add("clip_cond_proj.bias", H);
    add("text_input_proj.0.weight", H * s.text_dim);
    add("text_input_proj.0.bias", H);
    mlp("text_input_proj.2");
    add("text_cond_proj.weight", H * s.gtext_dim);
    add("text_cond_proj.bias", H);
    mlp("global_cond_mlp");
    return v;
}

struct CondWeights {
    std::vector<Tensor> m;
    std::vector<int64_t> off;
    const float *base;
    CondWeights(const orc_refcond_spec &s, const float *w) : m(cond_manifest(s)), base(w) {
        int64_t o = 0;
        for (const auto &t : m) { off.push_back(o); o += t.numel; }
    }
    const float *get(const std::string &name) const {
        for (size_t i = 0; i < m.size(); ++i)
            if (m[i].name == name) return base + off[i];
        fprintf(stderr, "oracle: missing tensor %s\n", name.c_str());
        abort();
    }
};

// convmlp (src/dit.cpp:14-20): y = w2 * (silu(w1 * x) . (w3 * x)), conv k3 pad 1, no bias
void convmlp(const CondWeights &W, const std::string &p, const float *x, float *y, int T, int C, int F) {
    std::vector<float> h1((size_t)T * F), h3((size_t)T * F);
    orc_conv1d(W.get(p + ".w1.weight"), nullptr, x, h1.data(), T, T, C, F, 3, 1, 1, 1);
    orc_conv1d(W.get(p + ".w3.weight"), nullptr, x, h3.data(), T, T, C, F, 3, 1, 1, 1);
    orc_swiglu(h1.data(), h3.data(), h1.data(), h1.size());
    orc_conv1d(W.get(p + ".w2.weight"), nullptr, h1.data(), y, T, T, F, C, 3, 1, 1, 1);
}

// mlp (src/dit.cpp:21-27): the same with linear layers
void mlp(const CondWeights &W, const std::string &p, const float *x, float *y, int rows, int C, int F) {
    std::vector<float> h1((size_t)rows * F), h3((size_t)rows * F);
    orc_gemm(W.get(p + ".w1.weight"), x, h1.data(), nullptr, rows, F, C, C, C, F);
    orc_gemm(W.get(p + ".w3.weight"), x, h3.data(), nullptr, rows, F, C, C, C, F);
    orc_swiglu(h1.data(), h3.data(), h1.data(), h1.size());
    orc_gemm(W.get(p + ".w2.weight"), h1.data(), y, nullptr, rows, C, F, F, F, C);
}

} // namespace

extern "C" int orc_refcond_manifest_count(const orc_refcond_spec *s) { return (int)cond_manifest(*s).size(); }
extern "C" int64_t orc_refcond_manifest_numel(const orc_refcond_spec *s, int idx) { return cond_manifest(*s)[idx].numel; }
extern "C" void orc_refcond_manifest_name(const orc_refcond_spec *s, int idx, char *buf, int cap) {
    snprintf(buf, cap, "%s", cond_manifest(*s)[idx].name.c_str());
}

extern "C" void orc_ref_prep_conditioning(const orc_refcond_spec *sp, const float *weights, const float *clip_f,
                                          const float *sync_f, float *clip_pp, float *sync_gather, float *clip_fc) {
    const orc_refcond_spec &s = *sp;
    const CondWeights W(s, weights);
    const int H = s.H, F = s.F, SS = s.sync_S, SD = s.sync_dim;
    // sync stream
    std::vector<float> sb((size_t)SS * SD), smid((size_t)SS * H);
    const float *pe = W.get("sync_pos_emb");
    for (int r = 0; r < SS; ++r)
        for (int c = 0; c < SD; ++c) sb[(size_t)r * SD + c] = sync_f[(size_t)r * SD + c] + pe[(size_t)(r % 8) * SD + c];
    orc_conv1d(W.get("sync_input_proj.0.weight"), W.get("sync_input_proj.0.bias"), sb.data(), smid.data(), SS, SS, SD,
               H, 7, 1, 3, 1);
    orc_silu(smid.data(), smid.size());
    convmlp(W, "sync_input_proj.2", smid.data(), smid.data(), SS, H, F);
    for (int i = 0; i < s.T; ++i) {
        const int si = (int)floorf(((float)i + 0.5f) * (float)SS / (float)s.T);
        memcpy(sync_gather + (size_t)i * H, smid.data() + (size_t)si * H, (size_t)H * sizeof(float));
    }
    // clip stream
    orc_gemm(W.get("clip_input_proj.0.weight"), clip_f, clip_pp, W.get("clip_input_proj.0.bias"), s.C, H, s.clip_dim,
             s.clip_dim, s.clip_dim, H);
    orc_silu(clip_pp, (size_t)s.C * H);
    convmlp(W, "clip_input_proj.2", clip_pp, clip_pp, s.C, H, F);
    std::vector<float> mean(H, 0.0f);
    for (int r = 0; r < s.C; ++r)
        for (int c = 0; c < H; ++c) mean[c] += clip_pp[(size_t)r * H + c];
    for (int c = 0; c < H; ++c) mean[c] /= (float)s.C;
    orc_gemv(W.get("clip_cond_proj.weight"), mean.data(), clip_fc, W.get("clip_cond_proj.bias"), H, H, H);
}

extern "C" void orc_ref_prep_text_arm(const orc_refcond_spec *sp, const float *weights, const float *text_cat,
                                      const float *gtext, const float *clip_fc, float *text_pp, float *gcmlp) {
    const orc_refcond_spec &s = *sp;
    const CondWeights W(s, weights);
    const int H = s.H, F = s.F;
    orc_gemm(W.get("text_input_proj.0.weight"), text_cat, text_pp, W.get("text_input_proj.0.bias"), s.TS, H,
             s.text_dim, s.text_dim, s.text_dim, H);
    orc_silu(text_pp, (size_t)s.TS * H);
    mlp(W, "text_input_proj.2", text_pp, text_pp, s.TS, H, F);
    std::vector<float> fc(H);
    orc_gemv(W.get("text_cond_proj.weight"), gtext, fc.data(), W.get("text_cond_proj.bias"), H, s.gtext_dim, s.gtext_dim);
    for (int c = 0; c < H; ++c) fc[c] += clip_fc[c];
    mlp(W, "global_cond_mlp", fc.data(), gcmlp, 1, H, F);
}
